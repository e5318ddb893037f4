// Channel modulation (HadamardChannelModulation, src/model/moe.py:610-771).
//
// Rows come in G groups of T rows each (the [B, T, C] input of the module;
// mHCLlamaBlock feeds it the [B*n, T, C] view of its [B, T, n, C] streams,
// mhc.py:528-532).  For group g:
//     bulk[g]  = mean_t xn[g, t]                       (moe.py:694)
//     h        = silu(W1 bulk[g]);  m = W2 h           (moe.py:697-700, :753-762)
//     scale_b  = 1 + clamp(temp, 0.1, 0.5) tanh(m_b);  shift_b = m_{nb + b}
//                                                       (moe.py:703-709)
//     out[c]   = xn[c] + r (xn[c] scale_b + 0.1 shift_b - xn[c]),  b = c / bd
//                                                       (moe.py:729-744, :116-153)
// where xn is the module input or, fused for the block (mhc.py:531,
// moe.py:796-798), RMSNorm(x) * w, with x + out written.
//
// Kernels (all sums in a fixed order: deterministic, no atomics):
//   colsum     per-column sums of a T-chunk of a group (the bulk state, or
//              in the backward the sums of g*x and g), one float partial per
//              (group, chunk); each wave keeps 1-8 rows' loads in flight;
//   mlp_fused  one 16-wave workgroup per group: the partials summed, then
//              both products of the MLP (used while hidden * C <= 2^19);
//   bulk + mlp the same in three launches for a wide MLP: partial sums,
//              then each product for 4 groups x 16 rows per workgroup (W1 /
//              W2 rows read once per workgroup, not once per group);
//   apply      RB rows per wave, per-column scale / shift / norm tables in
//              LDS built while the rows' loads are in flight;
//   bwd_reduce the backward's per-(group, block) sums of the partials.
// The colsum and the apply each read the input once: 2 reads + 1 write of
// it in all, HBM- (at small sizes latency-) bound.
#include "common.h"

namespace walsh {

constexpr int kCmWaves = 4;
constexpr int kCmThreads = 64 * kCmWaves;
constexpr int kCmMaxQ = 16;        // C <= 4096: up to 16 quads of 4 columns per lane
constexpr int kCmMaxC = 4 * 64 * kCmMaxQ;
constexpr int kCmMinChunk = 16;    // colsum: at least this many rows per workgroup

struct CmRows {
    const void *x;
    int64_t ldx;
    int G, T, C;
    const float *norm_w;   // nullable: rows are RMSNorm(x) * norm_w
    float eps;
};

template <int NQ>
__device__ __forceinline__ float row_rs(const f32x4 (&v)[NQ], int nq, int lane, int C, float eps) {
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
        if (lane + 64 * j >= nq) continue;
        sq += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    }
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) sq += __shfl_xor(sq, sh, 64);
    return 1.0f / sqrtf(__fdiv_rn(sq, (float)C) + eps);
}

// MODE 0: part[g][p][c] = sum over the chunk's rows of xn[c].
// MODE 1 (backward of the apply): part[g][p][0][c] = sum g*x, part[g][p][1][c]
//   = sum g, and gx = g * (1 + r (scale_b - 1)) is written on the way.
struct CmBwd {
    const void *gy;
    int64_t ldg;
    void *gx;
    int64_t ldgx;
    const float *scale;
    int64_t ld_ss;
    int bd;
    float r;
};

// Rows per wave per step: the loads of RB rows are issued before any is
// used, so several rows' memory latency overlaps.
template <int NQ> struct CmRB { static constexpr int value = NQ <= 2 ? 8 : NQ == 4 ? 4 : NQ == 8 ? 2 : 1; };
static inline int cm_rb(int nq) { return nq <= 2 ? 8 : nq == 4 ? 4 : nq == 8 ? 2 : 1; }

template <typename T, int MODE, int NQ>
__global__ __launch_bounds__(kCmThreads) void chanmod_colsum_kernel(CmRows a, CmBwd bw, int P, int chunk,
                                                                    float *__restrict__ part) {
    constexpr int RB = CmRB<NQ>::value;
    extern __shared__ float cm_smem[];  // [kCmWaves][C] reduction; MODE 1 also fac[C]
    const int p = blockIdx.x, g = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int C = a.C, nq = C >> 2;
    float *red = cm_smem;
    float *fac = cm_smem + kCmWaves * C;
    if (MODE == 1) {
        for (int c = threadIdx.x; c < C; c += kCmThreads) fac[c] = 1.0f + bw.r * (bw.scale[g * bw.ld_ss + c / bw.bd] - 1.0f);
        __syncthreads();
    }
    const int t0 = p * chunk;
    const int t1 = min(a.T, t0 + chunk);
    f32x4 acc0[NQ], acc1[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
        acc0[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc1[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    f32x4 nwv[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
        const int q = lane + 64 * j;
        nwv[j] = (MODE == 0 && a.norm_w) ? *(const f32x4 *)(a.norm_w + 4 * (q < nq ? q : nq - 1))
                                         : f32x4{1.f, 1.f, 1.f, 1.f};
    }
    for (int tb = t0 + wave * RB; tb < t1; tb += kCmWaves * RB) {
        f32x4 v[RB][NQ], gv[RB][NQ];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const bool ok = tb + r < t1;
            const int64_t row = (int64_t)g * a.T + (ok ? tb + r : t0);
            const T *xr = (const T *)a.x + row * a.ldx;
            const T *gr = MODE == 1 ? (const T *)bw.gy + row * bw.ldg : nullptr;
#pragma unroll
            for (int j = 0; j < NQ; ++j) {
                // unconditional loads from clamped (in-range) addresses, then
                // a select: a load under a branch would be waited on alone
                const int q = lane + 64 * j;
                const bool in = ok && q < nq;
                const int qc = q < nq ? q : nq - 1;
                const f32x4 xv = load4(xr + 4 * qc);
                v[r][j] = in ? xv : f32x4{0.f, 0.f, 0.f, 0.f};
                if (MODE == 1) {
                    const f32x4 g4 = load4(gr + 4 * qc);
                    gv[r][j] = in ? g4 : f32x4{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            if (tb + r >= t1) break;
            if (MODE == 0) {
                if (a.norm_w) {
                    const float rs = row_rs<NQ>(v[r], nq, lane, C, a.eps);
#pragma unroll
                    for (int j = 0; j < NQ; ++j) v[r][j] = v[r][j] * rs * nwv[j];
                }
#pragma unroll
                for (int j = 0; j < NQ; ++j) acc0[j] += v[r][j];
            } else {
                T *gxr = (T *)bw.gx + ((int64_t)g * a.T + tb + r) * bw.ldgx;
#pragma unroll
                for (int j = 0; j < NQ; ++j) {
                    const int q = lane + 64 * j;
                    if (q >= nq) continue;
                    acc0[j] += gv[r][j] * v[r][j];
                    acc1[j] += gv[r][j];
                    const f32x4 f = *(const f32x4 *)(fac + 4 * q);
                    store4(gxr + 4 * q, gv[r][j] * f);
                }
            }
        }
    }
    constexpr int NA = MODE == 0 ? 1 : 2;
#pragma unroll
    for (int k = 0; k < NA; ++k) {
        if (k) __syncthreads();  // red is reused
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            const int q = lane + 64 * j;
            if (q < nq) *(f32x4 *)(red + wave * C + 4 * q) = k ? acc1[j] : acc0[j];
        }
        __syncthreads();
        float *dst = part + (((int64_t)g * P + p) * NA + k) * C;
        for (int c = threadIdx.x; c < C; c += kCmThreads) {
            float s = red[c];
#pragma unroll
            for (int w = 1; w < kCmWaves; ++w) s += red[w * C + c];
            dst[c] = s;
        }
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) v += __shfl_xor(v, sh, 64);
    return v;
}

// bulk[g][c] = (sum over the P chunk partials, in chunk order) / T.  The
// partial loads are issued 8 at a time ahead of the adds.
__global__ __launch_bounds__(kCmThreads) void chanmod_bulk_kernel(const float *__restrict__ part, int P, int C, int T,
                                                                  float *__restrict__ bulk) {
    const int g = blockIdx.x;
    const float inv_t = 1.0f / (float)T;
    for (int c = threadIdx.x; c < C; c += kCmThreads) {
        const float *src = part + (int64_t)g * P * C + c;
        float s = 0.f;
        for (int p0 = 0; p0 < P; p0 += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = p0 + k < P ? src[(int64_t)(p0 + k) * C] : 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) s += v[k];
        }
        bulk[(int64_t)g * C + c] = s * inv_t;
    }
}

constexpr int kCmGT = 4;         // groups per MLP workgroup
constexpr int kCmRowsPerWg = 16; // MLP rows per workgroup (4 per wave)

// out[g][j] = act(sum_c w[j][c] in[g][c]) for a tile of kCmGT groups and
// kCmRowsPerWg rows j; the tile's inputs sit in LDS, each weight row is read
// once per workgroup.  act 0: silu -> out (stride ld_out);
// act 1: scale / shift -> ss (row j < nb: 1 + temp * tanh, else the value).
__global__ __launch_bounds__(kCmThreads) void chanmod_mlp_kernel(const float *__restrict__ in, int G, int K,
                                                                 const float *__restrict__ w, int rows, int act,
                                                                 float *__restrict__ out, int nb,
                                                                 const float *scale_temp) {
    extern __shared__ float cm_smem[];   // [kCmGT][K]
    const int g0 = blockIdx.x * kCmGT;
    const int ng = min(kCmGT, G - g0);
    for (int e = threadIdx.x; e < ng * K; e += kCmThreads) cm_smem[e] = in[(int64_t)g0 * K + e];
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float temp = act == 1 ? fminf(fmaxf(*scale_temp, 0.1f), 0.5f) : 0.f;
    for (int i = 0; i < kCmRowsPerWg / kCmWaves; ++i) {
        const int j = blockIdx.y * kCmRowsPerWg + wave * (kCmRowsPerWg / kCmWaves) + i;
        if (j >= rows) break;
        const float *wr = w + (int64_t)j * K;
        float d[kCmGT] = {0.f, 0.f, 0.f, 0.f};
        for (int c = lane; c < K; c += 64) {
            const float wv = wr[c];
#pragma unroll
            for (int gi = 0; gi < kCmGT; ++gi)
                if (gi < ng) d[gi] += wv * cm_smem[gi * K + c];
        }
#pragma unroll
        for (int gi = 0; gi < kCmGT; ++gi) {
            if (gi >= ng) continue;
            const float sv = wave_sum(d[gi]);
            if (lane == 0) {
                float o;
                if (act == 0) o = sv / (1.0f + expf(-sv));
                else o = j < nb ? 1.0f + temp * tanhf(sv) : sv;
                out[(int64_t)(g0 + gi) * rows + j] = o;
            }
        }
    }
}

// The whole scale / shift computation of one group in one workgroup of 16
// waves: bulk from the chunk partials, h = silu(W1 bulk), m = W2 h.  Used
// while W1 is small (hidden * C <= kCmFusedMax floats): a workgroup then
// reads all of it from L2 in a few microseconds, and three dependent
// launches become one.
constexpr int kCmMlpThreads = 1024;
constexpr int kCmMlpWaves = kCmMlpThreads / 64;
constexpr int64_t kCmFusedMax = 1 << 19;

__global__ __launch_bounds__(kCmMlpThreads) void chanmod_mlp_fused_kernel(const float *__restrict__ part, int P, int C,
                                                                          int T, const float *__restrict__ w1,
                                                                          int hidden, const float *__restrict__ w2,
                                                                          int nb, const float *scale_temp,
                                                                          float *__restrict__ ss) {
    extern __shared__ float cm_smem[];   // bulk [C], h [hidden]
    float *bulk = cm_smem, *hl = cm_smem + C;
    const int g = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float inv_t = 1.0f / (float)T;
    for (int c = tid; c < C; c += kCmMlpThreads) {
        const float *src = part + (int64_t)g * P * C + c;
        float s = 0.f;
        for (int p0 = 0; p0 < P; p0 += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = p0 + k < P ? src[(int64_t)(p0 + k) * C] : 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) s += v[k];
        }
        bulk[c] = s * inv_t;
    }
    __syncthreads();
    // layer 1: 4 rows per wave at a time, 16-byte weight loads
    constexpr int R = 4;
    const int c4n = C >> 2;
    for (int j0 = wave; j0 < hidden; j0 += kCmMlpWaves * R) {
        float d[R] = {0.f, 0.f, 0.f, 0.f};
        for (int c4 = lane; c4 < c4n; c4 += 64) {
            const f32x4 b = *(const f32x4 *)(bulk + 4 * c4);
            f32x4 w[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int j = j0 + kCmMlpWaves * r;
                w[r] = j < hidden ? *(const f32x4 *)(w1 + (int64_t)j * C + 4 * c4) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int r = 0; r < R; ++r) d[r] += w[r].x * b.x + w[r].y * b.y + w[r].z * b.z + w[r].w * b.w;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int j = j0 + kCmMlpWaves * r;
            const float sv = wave_sum(d[r]);
            if (lane == 0 && j < hidden) hl[j] = sv / (1.0f + expf(-sv));
        }
    }
    __syncthreads();
    const float temp = fminf(fmaxf(*scale_temp, 0.1f), 0.5f);
    for (int k = wave; k < 2 * nb; k += kCmMlpWaves) {
        const float *wr = w2 + (int64_t)k * hidden;
        float d = 0.f;
        for (int c = lane; c < hidden; c += 64) d += wr[c] * hl[c];
        const float sv = wave_sum(d);
        if (lane == 0) ss[(int64_t)g * 2 * nb + k] = k < nb ? 1.0f + temp * tanhf(sv) : sv;
    }
}

struct CmApply {
    CmRows rows;
    void *y;
    int64_t ldy;
    const float *scale, *shift;
    int64_t ld_ss;
    int bd;
    float r, shift_scale;
    int add_input;
};

template <typename T, int NQ>
__global__ __launch_bounds__(kCmThreads) void chanmod_apply_kernel(CmApply a) {
    // one batch of RB rows per wave; the rows' loads are issued before the
    // per-column tables are built, so both latencies overlap
    constexpr int RB = CmRB<NQ>::value;
    extern __shared__ float cm_smem[];
    const CmRows &rw = a.rows;
    const int C = rw.C, nq = C >> 2;
    const int g = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tb = (blockIdx.x * kCmWaves + wave) * RB;
    f32x4 v[RB][NQ];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int t = tb + r;
        const bool ok = t < rw.T;
        const T *xr = (const T *)rw.x + ((int64_t)g * rw.T + (ok ? t : 0)) * rw.ldx;
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            const int q = lane + 64 * j;
            const f32x4 xv = load4(xr + 4 * (q < nq ? q : nq - 1));   // clamped, unconditional
            v[r][j] = ok && q < nq ? xv : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    float *sc = cm_smem, *sh = cm_smem + C, *nw = cm_smem + 2 * C;
    for (int c = threadIdx.x; c < C; c += kCmThreads) {
        const int b = c / a.bd;
        sc[c] = a.scale[g * a.ld_ss + b];
        sh[c] = a.shift[g * a.ld_ss + b];
        nw[c] = rw.norm_w ? rw.norm_w[c] : 1.0f;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int t = tb + r;
        if (t >= rw.T) break;
        T *yr = (T *)a.y + ((int64_t)g * rw.T + t) * a.ldy;
        const float rs = rw.norm_w ? row_rs<NQ>(v[r], nq, lane, C, rw.eps) : 1.0f;
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            const int q = lane + 64 * j;
            if (q >= nq) continue;
            const f32x4 s = *(const f32x4 *)(sc + 4 * q), h = *(const f32x4 *)(sh + 4 * q);
            f32x4 xn = v[r][j];
            if (rw.norm_w) xn = xn * rs * *(const f32x4 *)(nw + 4 * q);
            const f32x4 xm = xn * s + h * a.shift_scale;
            f32x4 o = xn + a.r * (xm - xn);
            if (a.add_input) o = v[r][j] + o;
            store4(yr + 4 * q, o);
        }
    }
}

// grad_scale[g][b] = r * sum (g x) over the group's rows and block b's columns;
// grad_shift[g][b] = shift_scale * r * sum g (moe.py:155-199).
__global__ __launch_bounds__(64) void chanmod_bwd_reduce_kernel(const float *__restrict__ part, int P, int C, int nb,
                                                                int bd, float r, float shift_scale, float *dscale,
                                                                float *dshift, int64_t ld_ss) {
    const int g = blockIdx.x;
    for (int b = threadIdx.x; b < nb; b += 64) {
        float s0 = 0.f, s1 = 0.f;
        for (int p = 0; p < P; ++p) {
            const float *src = part + ((int64_t)g * P + p) * 2 * C + b * bd;
            for (int c = 0; c < bd; ++c) {
                s0 += src[c];
                s1 += src[C + c];
            }
        }
        dscale[g * ld_ss + b] = s0 * r;
        dshift[g * ld_ss + b] = s1 * shift_scale * r;
    }
}

static int cm_split(int64_t G, int64_t T, int *chunk) {
    int64_t P = ceil_div((int64_t)device_info().cu_count * 2, G);
    const int64_t maxP = ceil_div(T, kCmMinChunk);
    if (P > maxP) P = maxP;
    if (P < 1) P = 1;
    *chunk = (int)ceil_div(T, P);
    return (int)ceil_div(T, *chunk);
}

static int cm_check_rows(const char *fn, const void *x, int64_t ldx, int64_t G, int64_t T, int64_t C, int dtype) {
    if (G < 0 || T < 0 || G > 65535 || T > (1 << 30))
        return set_error(WALSH_EINVAL, "%s: bad shape G=%lld T=%lld", fn, (long long)G, (long long)T);
    if (C < 4 || C > kCmMaxC || C % 4)
        return set_error(WALSH_ENOTSUP, "%s: C=%lld (a multiple of 4 up to %d)", fn, (long long)C, kCmMaxC);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d", fn, dtype);
    const int64_t align = dtype == WALSH_BF16 ? 8 : 16;
    if (ldx < C || ldx % 4 || (uintptr_t)x % align)
        return set_error(WALSH_ENOTSUP, "%s: rows must be %lld-byte aligned with a stride multiple of 4", fn,
                         (long long)align);
    return WALSH_OK;
}

// Quads of 4 columns per lane the kernels are built for: 2, 4, 8 or 16.
static int cm_nq(int64_t C) {
    const int64_t q = ceil_div(C, 4 * 64);
    return q <= 2 ? 2 : q <= 4 ? 4 : q <= 8 ? 8 : 16;
}

template <typename T, int MODE>
static void cm_colsum(int nq, dim3 g, uint32_t lds, hipStream_t s, const CmRows &rows, const CmBwd &bw, int P,
                      int chunk, float *part) {
    if (nq == 2) launch(chanmod_colsum_kernel<T, MODE, 2>, g, dim3(kCmThreads), lds, s, rows, bw, P, chunk, part);
    else if (nq == 4) launch(chanmod_colsum_kernel<T, MODE, 4>, g, dim3(kCmThreads), lds, s, rows, bw, P, chunk, part);
    else if (nq == 8) launch(chanmod_colsum_kernel<T, MODE, 8>, g, dim3(kCmThreads), lds, s, rows, bw, P, chunk, part);
    else launch(chanmod_colsum_kernel<T, MODE, 16>, g, dim3(kCmThreads), lds, s, rows, bw, P, chunk, part);
}

template <typename T>
static void cm_apply(int nq, dim3 g, uint32_t lds, hipStream_t s, const CmApply &ap) {
    if (nq == 2) launch(chanmod_apply_kernel<T, 2>, g, dim3(kCmThreads), lds, s, ap);
    else if (nq == 4) launch(chanmod_apply_kernel<T, 4>, g, dim3(kCmThreads), lds, s, ap);
    else if (nq == 8) launch(chanmod_apply_kernel<T, 8>, g, dim3(kCmThreads), lds, s, ap);
    else launch(chanmod_apply_kernel<T, 16>, g, dim3(kCmThreads), lds, s, ap);
}

}  // namespace walsh

using namespace walsh;

// Workspace: bulk [G][C] then the chunk partials [G][P][2][C]; the MLP's
// hidden activations [G][hidden] (hidden <= 2C) reuse the partials' space
// once the bulk state is formed.
WALSH_EXPORT int64_t walsh_chanmod_workspace_bytes(int64_t G, int64_t T, int64_t C) {
    if (G <= 0 || T <= 0 || C <= 0) return 0;
    int chunk;
    const int P = cm_split(G, T, &chunk);
    return (G * C + G * P * 2 * C) * (int64_t)sizeof(float);
}

WALSH_EXPORT int walsh_chanmod_fwd(const void *x, int64_t ldx, int64_t G, int64_t T, int64_t C, const float *norm_w,
                                   float eps, const float *w1, int64_t hidden, const float *w2, int64_t n_blocks,
                                   const float *scale_temp, float residual_scale, float shift_scale, int add_input,
                                   void *y, int64_t ldy, float *scale_shift, int dtype, void *workspace,
                                   int64_t workspace_bytes, void *stream) {
    const char *fn = "walsh_chanmod_fwd";
    int rc = cm_check_rows(fn, x, ldx, G, T, C, dtype);
    if (rc) return rc;
    if (G == 0 || T == 0) return WALSH_OK;
    if (!x || !w1 || !w2 || !scale_temp || !y || !scale_shift || !workspace)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (n_blocks < 1 || C % n_blocks || hidden < 1 || hidden > 2 * C)
        return set_error(WALSH_EINVAL, "%s: n_blocks=%lld hidden=%lld for C=%lld (hidden <= 2C)", fn,
                         (long long)n_blocks, (long long)hidden, (long long)C);
    const int64_t align = dtype == WALSH_BF16 ? 8 : 16;
    if (ldy < C || ldy % 4 || (uintptr_t)y % align) return set_error(WALSH_ENOTSUP, "%s: output alignment", fn);
    if (norm_w && (uintptr_t)norm_w % 16) return set_error(WALSH_ENOTSUP, "%s: norm weight alignment", fn);
    int chunk;
    const int P = cm_split(G, T, &chunk);
    if (workspace_bytes < walsh_chanmod_workspace_bytes(G, T, C))
        return set_error(WALSH_EINVAL, "%s: workspace too small", fn);
    const int64_t lds_mlp = kCmGT * (C > hidden ? C : hidden) * (int64_t)sizeof(float);
    if (lds_mlp > device_info().max_shared_per_block)
        return set_error(WALSH_ENOTSUP, "%s: C / hidden too large for LDS", fn);
    hipStream_t s = (hipStream_t)stream;
    float *bulk = (float *)workspace;
    float *part = bulk + G * C;
    float *hid = part;   // after the bulk kernel has consumed the partials
    CmRows rows{x, ldx, (int)G, (int)T, (int)C, norm_w, eps};
    const CmBwd nob{};
    const dim3 gc((unsigned)P, (unsigned)G);
    const uint32_t lds_c = (uint32_t)(kCmWaves * C * sizeof(float));
    const int nq = cm_nq(C);
    if (dtype == WALSH_BF16) cm_colsum<uint16_t, 0>(nq, gc, lds_c, s, rows, nob, P, chunk, part);
    else cm_colsum<float, 0>(nq, gc, lds_c, s, rows, nob, P, chunk, part);
    if (hidden * C <= kCmFusedMax && (uintptr_t)w1 % 16 == 0) {
        launch(chanmod_mlp_fused_kernel, dim3((unsigned)G), dim3(kCmMlpThreads), (uint32_t)((C + hidden) * sizeof(float)),
               s, (const float *)part, P, (int)C, (int)T, w1, (int)hidden, w2, (int)n_blocks, scale_temp, scale_shift);
    } else {
        launch(chanmod_bulk_kernel, dim3((unsigned)G), dim3(kCmThreads), 0, s, (const float *)part, P, (int)C,
               (int)T, bulk);
        const unsigned gtiles = (unsigned)ceil_div(G, kCmGT);
        launch(chanmod_mlp_kernel, dim3(gtiles, (unsigned)ceil_div(hidden, kCmRowsPerWg)), dim3(kCmThreads),
               (uint32_t)(kCmGT * C * sizeof(float)), s, (const float *)bulk, (int)G, (int)C, w1, (int)hidden, 0, hid,
               (int)n_blocks, scale_temp);
        launch(chanmod_mlp_kernel, dim3(gtiles, (unsigned)ceil_div(2 * n_blocks, kCmRowsPerWg)), dim3(kCmThreads),
               (uint32_t)(kCmGT * hidden * sizeof(float)), s, (const float *)hid, (int)G, (int)hidden, w2,
               (int)(2 * n_blocks), 1, scale_shift, (int)n_blocks, scale_temp);
    }
    CmApply ap{rows, y, ldy, scale_shift, scale_shift + n_blocks, 2 * n_blocks, (int)(C / n_blocks), residual_scale,
               shift_scale, add_input};
    const dim3 ga((unsigned)ceil_div(T, kCmWaves * cm_rb(cm_nq(C))), (unsigned)G);
    const uint32_t lds_a = (uint32_t)(3 * C * sizeof(float));
    if (dtype == WALSH_BF16) cm_apply<uint16_t>(nq, ga, lds_a, s, ap);
    else cm_apply<float>(nq, ga, lds_a, s, ap);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_chanmod_apply(const void *x, int64_t ldx, int64_t G, int64_t T, int64_t C, int64_t n_blocks,
                                     const float *scale, const float *shift, int64_t ld_ss, float residual_scale,
                                     float shift_scale, void *y, int64_t ldy, int dtype, void *stream) {
    const char *fn = "walsh_chanmod_apply";
    int rc = cm_check_rows(fn, x, ldx, G, T, C, dtype);
    if (rc) return rc;
    if (G == 0 || T == 0) return WALSH_OK;
    if (!x || !scale || !shift || !y) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (n_blocks < 1 || C % n_blocks || ld_ss < n_blocks)
        return set_error(WALSH_EINVAL, "%s: n_blocks=%lld ld=%lld for C=%lld", fn, (long long)n_blocks,
                         (long long)ld_ss, (long long)C);
    const int64_t align = dtype == WALSH_BF16 ? 8 : 16;
    if (ldy < C || ldy % 4 || (uintptr_t)y % align) return set_error(WALSH_ENOTSUP, "%s: output alignment", fn);
    CmApply ap{CmRows{x, ldx, (int)G, (int)T, (int)C, nullptr, 0.f}, y, ldy, scale, shift, ld_ss,
               (int)(C / n_blocks), residual_scale, shift_scale, 0};
    hipStream_t s = (hipStream_t)stream;
    const dim3 ga((unsigned)ceil_div(T, kCmWaves * cm_rb(cm_nq(C))), (unsigned)G);
    const uint32_t lds_a = (uint32_t)(3 * C * sizeof(float));
    if (dtype == WALSH_BF16) cm_apply<uint16_t>(cm_nq(C), ga, lds_a, s, ap);
    else cm_apply<float>(cm_nq(C), ga, lds_a, s, ap);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_chanmod_bwd(const void *gy, int64_t ldg, const void *x, int64_t ldx, int64_t G, int64_t T,
                                   int64_t C, int64_t n_blocks, const float *scale, int64_t ld_ss,
                                   float residual_scale, float shift_scale, void *gx, int64_t ldgx, float *dscale,
                                   float *dshift, int dtype, void *workspace, int64_t workspace_bytes, void *stream) {
    const char *fn = "walsh_chanmod_bwd";
    int rc = cm_check_rows(fn, x, ldx, G, T, C, dtype);
    if (!rc) rc = cm_check_rows(fn, gy, ldg, G, T, C, dtype);
    if (!rc) rc = cm_check_rows(fn, gx, ldgx, G, T, C, dtype);
    if (rc) return rc;
    if (G == 0) return WALSH_OK;
    if (!scale || !dscale || !dshift) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (n_blocks < 1 || C % n_blocks || ld_ss < n_blocks)
        return set_error(WALSH_EINVAL, "%s: n_blocks=%lld ld=%lld for C=%lld", fn, (long long)n_blocks,
                         (long long)ld_ss, (long long)C);
    hipStream_t s = (hipStream_t)stream;
    if (T == 0) {
        // no rows: the sums are empty (the reduce over zero partials writes zeros)
        launch(chanmod_bwd_reduce_kernel, dim3((unsigned)G), dim3(64), 0, s, (const float *)nullptr, 0, (int)C,
               (int)n_blocks, (int)(C / n_blocks), residual_scale, shift_scale, dscale, dshift, ld_ss);
        return check_hip(hipGetLastError(), fn);
    }
    if (!x || !gy || !gx || !workspace) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    int chunk;
    const int P = cm_split(G, T, &chunk);
    if (workspace_bytes < G * P * 2 * C * (int64_t)sizeof(float))
        return set_error(WALSH_EINVAL, "%s: workspace too small", fn);
    float *part = (float *)workspace;
    const int bd = (int)(C / n_blocks);
    CmRows rows{x, ldx, (int)G, (int)T, (int)C, nullptr, 0.f};
    CmBwd bw{gy, ldg, gx, ldgx, scale, ld_ss, bd, residual_scale};
    const dim3 gc((unsigned)P, (unsigned)G);
    const uint32_t lds_c = (uint32_t)((kCmWaves + 1) * C * sizeof(float));
    if (dtype == WALSH_BF16) cm_colsum<uint16_t, 1>(cm_nq(C), gc, lds_c, s, rows, bw, P, chunk, part);
    else cm_colsum<float, 1>(cm_nq(C), gc, lds_c, s, rows, bw, P, chunk, part);
    launch(chanmod_bwd_reduce_kernel, dim3((unsigned)G), dim3(64), 0, s, (const float *)part, P, (int)C,
           (int)n_blocks, bd, residual_scale, shift_scale, dscale, dshift, ld_ss);
    return check_hip(hipGetLastError(), fn);
}
