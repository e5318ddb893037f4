// Hadamard-32 ternary linear backward: the autograd of HadamardLinear.forward
// (src/model/fht_cuda.py:489-519) with FHTFunction's self-adjoint backward
// (fht_cuda.py:328-332) and physics.quantize_ternary's straight-through
// estimator (src/model/physics.py:43-50).
//
// Forward (H = H0 / sqrt(32), H0 the +-1 Sylvester matrix over the 32 groups):
//   y = beta .* H W H (alpha .* x)
// Backward for an output gradient gy:
//   dx     = alpha .* (H W^T H (beta .* gy))          (a forward pass of the
//            transposed layer: input gy, alpha' = beta, beta' = alpha)
//   dalpha = sum_rows x .* H W^T H (beta .* gy)
//   dbeta  = sum_rows gy .* H W H (alpha .* x)
//   dW_g   = sum_rows H(beta .* gy)_g (outer) H(alpha .* x)_g
//   dlatent = dW .* [|latent| <= 1.5]                  (the clamp of the STE:
//            w_clamped + (w_quant - w_clamped).detach() passes gradient only
//            through w.clamp(-1.5, 1.5))
// Every product above is H0 ... H0 / 32, so the kernels run unnormalised
// transforms and the reduction applies the 1/32.
//
// Kernel: hadamard_bwd_kernel, one launch with three workgroup roles.
//   dW role: per (token range, output tile, input chunk), H0(beta .* gy) and
//     H0(alpha .* x) in the forward lane layout (lane = token, 4 columns),
//     turned into token-major fragments by a matrix-core product with the
//     identity, then dW_g += dyp_g^T xm_g on matrix cores with the 16 tokens
//     of a tile as the contraction.  The four waves of a workgroup add their
//     dW in LDS in a fixed order and write one partial.
//   dx / dalpha role and dbeta role: a forward-style pass (transform,
//     ternary contraction on matrix cores, transform) whose epilogue
//     multiplies the result by an auxiliary row tensor and keeps per-lane
//     sums over the wave's tiles (dalpha with aux = x while storing dx;
//     dbeta with aux = gy, no store); a wave's sums are reduced over its 16
//     token lanes with DPP row rotations and written as one partial row.
// hadamard_bwd_reduce_kernel: fixed-order column sums of the partials, the
//   1/32 and the STE mask.
// All sums run in a fixed order: results are identical from run to run.
#include "hadamard_core.h"

namespace walsh {

// ---------------------------------------------------------------- weights

// Reference packing (4 codes per byte along K, byte = v0<<6|v1<<4|v2<<2|v3,
// v = code + 1; fht_cuda.py:65-93) of the transposed codes:
// packed_t[g][i][o/4] from packed[g][o][i/4].
__global__ void hadamard_pack_transpose_kernel(const uint8_t *__restrict__ packed, int in_o, int out_o,
                                               uint8_t *__restrict__ packed_t) {
    const int kp4 = (int)ceil_div(in_o, 4), op4 = (int)ceil_div(out_o, 4);
    const int64_t total = (int64_t)32 * in_o * op4;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int ob = (int)(e % op4);
        const int64_t gi = e / op4;
        const int i = (int)(gi % in_o), g = (int)(gi / in_o);
        uint32_t b = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int o = 4 * ob + j;
            uint32_t v = 1u;  // code 0 past out_o
            if (o < out_o) v = (packed[((int64_t)g * out_o + o) * kp4 + i / 4] >> (6 - 2 * (i & 3))) & 3u;
            b |= v << (6 - 2 * j);
        }
        packed_t[e] = (uint8_t)b;
    }
}

// ---------------------------------------------------------------- helpers

// Sum over the 16 lanes of each DPP row (lanes 16r .. 16r+15): rotations by
// 8, 4, 2, 1 leave every lane of the row holding the row's total.
__device__ __forceinline__ float row_sum16(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
    return v;
}

// LDS scale table [nc][4][32] f32x4: entry (c*4 + q)*32 + g holds
// s[g][16c + 4q .. +3] (zeros past n), the layout load_transform reads.
__device__ __forceinline__ void fill_scale(f32x4 *__restrict__ dst, const float *__restrict__ s, int n, int nc,
                                           float mul, int tid, int nthreads) {
    for (int e = tid; e < nc * 128; e += nthreads) {
        const int g = e & 31, i0 = 4 * (e >> 5);
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (i0 + j < n) ? (s ? s[g * n + i0 + j] : 1.f) * mul : 0.f;
        dst[e] = v;
    }
}

__device__ __forceinline__ void fill_lut(void *lut, bool bf16, int tid) {
    const uint32_t byte = (uint32_t)tid;  // 256 threads, 256 entries
    float val[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) val[j] = (float)((int)((byte >> (6 - 2 * j)) & 3u) - 1);
    if (bf16) {
        uint2 e;
        e.x = pack_bf16x2(val[0], val[1]);
        e.y = pack_bf16x2(val[2], val[3]);
        ((uint2 *)lut)[byte] = e;
    } else {
        ((f32x4 *)lut)[byte] = f32x4{val[0], val[1], val[2], val[3]};
    }
}

// ---------------------------------------------------------------- reduce-epilogue pass

struct BwdRed {
    const void *aux;  // rows of the auxiliary tensor, laid out like the output
    int64_t ld_aux;
    int gs_aux;       // group stride of aux rows
    float *part;      // [S][32][Nt * 16] per-wave sums of (H0 W H0 (alpha .* in)) .* aux
    int S, tps;       // splits of the tile range, tiles per split
};

template <typename T, bool BF16MMA, bool VEC, bool STORE>
__device__ __forceinline__ void bwd_red_role(const HadArgs &a, const BwdRed &r, int blk, unsigned char *smem) {
    void *lut = smem;
    f32x4 *alpha_l = (f32x4 *)(smem + lut_bytes<BF16MMA>());
    f32x4 *beta_l = alpha_l + a.Kc * 128;
    const int tid = threadIdx.x;
    fill_lut(lut, BF16MMA, tid);
    fill_scale(alpha_l, a.alpha, a.in_o, a.Kc, 1.f, tid, kThreads);
    if (STORE) fill_scale(beta_l, a.beta, a.out_o, a.Nt, 0.03125f, tid, kThreads);
    __syncthreads();

    constexpr uint32_t esz = sizeof(T);
    const int wave = tid >> 6, lane = tid & 63, t = lane & 15, q = lane >> 4;
    const int wid = blk * kWaves + wave;
    if (wid >= r.S * a.Nt) return;  // no barrier follows
    const int nt = wid % a.Nt, s = wid / a.Nt;
    const int n_tiles = (int)ceil_div(a.M, kTile);
    const int t0 = s * r.tps;
    const int t1 = t0 + r.tps < n_tiles ? t0 + r.tps : n_tiles;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a, esz));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, STORE ? (uint32_t)((int64_t)a.M * a.ldy * esz) : 0u);
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(r.aux, (uint32_t)((int64_t)a.M * r.ld_aux * esz));
    const int o0 = kNTile * nt + 4 * q;
    const uint32_t astride = (uint32_t)r.gs_aux * esz;

    f32x4 red[32];
#pragma unroll
    for (int h = 0; h < 32; ++h) red[h] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int tile = t0; tile < t1; ++tile) {
        const int row = tile * kTile + t;
        const bool row_ok = row < a.M;
        const uint32_t xoff = row_ok ? x_row_off(a, row, esz) : 0u;
        f32x4 acc[32];
#pragma unroll
        for (int g = 0; g < 32; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < a.Kc; ++c) {
            XM<BF16MMA> xm;
            load_transform<T, BF16MMA, VEC>(a, xr, xoff, row_ok, c, q, alpha_l, xm);
            contract<BF16MMA>(a, nt, c, lane, xm, lut, acc);
        }
        fht32x4(acc);
        const uint32_t aoff = (uint32_t)((int64_t)row * r.ld_aux * esz);
        if (VEC) {
            const uint32_t voff = (row_ok && o0 < a.out_o) ? aoff + (uint32_t)o0 * esz : kOOB;
#pragma unroll
            for (int h = 0; h < 32; ++h) {
                red[h] += acc[h] * Buf4<T>::load(ar, voff, (uint32_t)h * astride);
                if ((h & 7) == 7) __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            uint32_t voff[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) voff[j] = (row_ok && o0 + j < a.out_o) ? aoff + (uint32_t)(o0 + j) * esz : kOOB;
#pragma unroll
            for (int h = 0; h < 32; ++h) {
#pragma unroll
                for (int j = 0; j < 4; ++j) red[h][j] += acc[h][j] * Buf4<T>::load1(ar, voff[j], (uint32_t)h * astride);
                if ((h & 7) == 7) __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (STORE) {
            const uint32_t yoff = (uint32_t)((int64_t)row * a.ldy * esz);
            transform_store<T, VEC, false>(a, acc, yr, yoff, row_ok, nt, q, beta_l, row);
        }
    }

    const int W = a.Nt * kNTile;
    float *dst = r.part + (int64_t)s * 32 * W + o0;
#pragma unroll
    for (int h = 0; h < 32; ++h) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = row_sum16(red[h][j]);
        if (t == 0) *(f32x4 *)(dst + (int64_t)h * W) = v;
    }
}

// ---------------------------------------------------------------- dW pass

struct BwdDW {
    float *part;  // [S][32][Nt*16][Kc*16] per-workgroup sums of dyp (outer) xm
    int S, tps;   // splits of the tile range (workgroups per (nt, c)), tiles per split
};

// 16x16 tile of (token, column) values in the forward lane layout (lane
// (t, q) holds columns 4q..4q+3 of token t) -> token-major fragments (lane
// (n, kq) holds tokens 4kq..4kq+3 of column n): D = A * I on the matrix
// cores with A = the tile, exact since every product is by 1 or 0.
__device__ __forceinline__ uint2 transpose_bf16(uint2 tile, uint2 ident) {
    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, tile),
                                                               __builtin_bit_cast(i16x4, ident),
                                                               f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    uint2 o;
    o.x = pack_bf16x2(d[0], d[1]);
    o.y = pack_bf16x2(d[2], d[3]);
    return o;
}
__device__ __forceinline__ f32x4 transpose_f32(f32x4 tile, f32x4 ident) {
    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) d = __builtin_amdgcn_mfma_f32_16x16x4f32(tile[s], ident[s], d, 0, 0, 0);
    return d;
}

template <typename T, bool BF16MMA, bool VEC>
__device__ __forceinline__ void bwd_dw_role(const HadArgs &ax, const HadArgs &ag, const BwdDW &d, int blk,
                                            unsigned char *smem) {
    f32x4 *alpha_l = (f32x4 *)smem;             // [Kc][4][32]
    f32x4 *beta_l = alpha_l + ax.Kc * 128;      // [Nt][4][32]
    f32x4 *sum_l = beta_l + ag.Kc * 128;        // [32][64]
    const int tid = threadIdx.x;
    fill_scale(alpha_l, ax.alpha, ax.in_o, ax.Kc, 1.f, tid, kThreads);
    fill_scale(beta_l, ag.alpha, ag.in_o, ag.Kc, 1.f, tid, kThreads);
    __syncthreads();

    constexpr uint32_t esz = sizeof(T);
    const int wave = tid >> 6, lane = tid & 63, t = lane & 15, q = lane >> 4;
    const int Kc = ax.Kc, Nt = ag.Kc;
    const int item = blk;
    const int c = item % Kc, nt = (item / Kc) % Nt, s = item / (Kc * Nt);
    const int n_tiles = (int)ceil_div(ax.M, kTile);
    const int t0 = s * d.tps;
    const int t1 = t0 + d.tps < n_tiles ? t0 + d.tps : n_tiles;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(ax.x, x_bytes(ax, esz));
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(ag.x, x_bytes(ag, esz));

    // identity B fragments: lane (n, kq) holds I[4kq + j][n]
    const int n = lane & 15, kq = lane >> 4;
    uint2 id_b;
    f32x4 id_f;
    if constexpr (BF16MMA) {
        id_b.x = (4 * kq + 0 == n ? 0x3f80u : 0u) | (4 * kq + 1 == n ? 0x3f800000u : 0u);
        id_b.y = (4 * kq + 2 == n ? 0x3f80u : 0u) | (4 * kq + 3 == n ? 0x3f800000u : 0u);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) id_f[j] = (4 * kq + j == n) ? 1.f : 0.f;
    }

    f32x4 dw[32];
#pragma unroll
    for (int g = 0; g < 32; ++g) dw[g] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int tile = t0 + wave; tile < t1; tile += kWaves) {
        const int row = tile * kTile + t;
        const bool row_ok = row < ax.M;
        XM<BF16MMA> gm;
        load_transform<T, BF16MMA, VEC>(ag, gr, row_ok ? x_row_off(ag, row, esz) : 0u, row_ok, nt, q, beta_l, gm);
        XM<BF16MMA> gt;
#pragma unroll
        for (int g = 0; g < 32; ++g) {
            if constexpr (BF16MMA) gt.b[g] = transpose_bf16(gm.b[g], id_b);
            else gt.v[g] = transpose_f32(gm.v[g], id_f);
        }
        XM<BF16MMA> xm;
        load_transform<T, BF16MMA, VEC>(ax, xr, row_ok ? x_row_off(ax, row, esz) : 0u, row_ok, c, q, alpha_l, xm);
#pragma unroll
        for (int g = 0; g < 32; ++g) {
            if constexpr (BF16MMA) {
                const uint2 xt = transpose_bf16(xm.b[g], id_b);
                dw[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, gt.b[g]),
                                                                   __builtin_bit_cast(i16x4, xt), dw[g], 0, 0, 0);
            } else {
                const f32x4 xt = transpose_f32(xm.v[g], id_f);
#pragma unroll
                for (int k = 0; k < 4; ++k) dw[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(gt.v[g][k], xt[k], dw[g], 0, 0, 0);
            }
            if ((g & 7) == 7) __builtin_amdgcn_sched_barrier(0);
        }
    }

    // waves add into LDS in order 0, 1, 2, 3 (uniform barriers)
    for (int w = 0; w < kWaves; ++w) {
        if (wave == w) {
#pragma unroll
            for (int g = 0; g < 32; ++g) sum_l[g * 64 + lane] = w == 0 ? dw[g] : sum_l[g * 64 + lane] + dw[g];
        }
        __syncthreads();
    }
    // lane (n, mq) of entry (g, lane) holds dW_g[o = 16nt + 4mq + j][i = 16c + n]
    const int Op = Nt * kNTile, Ip = Kc * kKChunk;
    float *dst = d.part + (int64_t)s * 32 * Op * Ip;
    for (int e = tid; e < 32 * 64; e += kThreads) {
        const int g = e >> 6, l = e & 63;
        const f32x4 v = sum_l[e];
        const int i = kKChunk * c + (l & 15), ob = kNTile * nt + 4 * (l >> 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[((int64_t)g * Op + ob + j) * Ip + i] = v[j];
    }
}

// ---------------------------------------------------------------- one launch, three roles

// The three passes read the same rows and are independent, so they run as
// one launch: workgroups [0, nW) take the dW role, the next nA the dx/dalpha
// role, the last nB the dbeta role (the longest role first, so its
// workgroups are dispatched first).
struct BwdJob {
    HadArgs a;   // transposed layer on gy (dx / dalpha)
    BwdRed ra;
    HadArgs b;   // the layer on x (dbeta)
    BwdRed rb;
    HadArgs wx, wg;  // x and gy as transform inputs (dW)
    BwdDW dw;
    int nW, nA, nB;
};

template <typename T, bool BF16MMA, bool VEC, bool STORE>
__global__ __launch_bounds__(kThreads, 1) void hadamard_bwd_kernel(BwdJob j) {
    extern __shared__ __align__(16) unsigned char smem[];
    int blk = blockIdx.x;
    if (blk < j.nW) {
        bwd_dw_role<T, BF16MMA, VEC>(j.wx, j.wg, j.dw, blk, smem);
        return;
    }
    blk -= j.nW;
    if (blk < j.nA) {
        bwd_red_role<T, BF16MMA, VEC, STORE>(j.a, j.ra, blk, smem);
        return;
    }
    bwd_red_role<T, BF16MMA, VEC, false>(j.b, j.rb, blk - j.nA, smem);
}

// ---------------------------------------------------------------- final reduction

struct BwdSum {
    const float *pa;  // [Sa][32][Ap]  dalpha partials
    const float *pb;  // [Sb][32][Bp]  dbeta partials
    const float *pw;  // [Sw][32][Op][Ip]  dW partials
    int Sa, Ap, Sb, Bp, Sw, Op, Ip;
    int in_o, out_o;
    const float *latent;  // [32][out_o][in_o] latent weights (STE mask), or null
    float *da, *db, *dw;  // null: not wanted
};

constexpr int kSumCols = 64;     // partial columns per workgroup
constexpr int kSumPhases = 16;   // partial rows summed in parallel, s = phase mod 16

__host__ __device__ inline int64_t sum_blocks(const BwdSum &r, int64_t *bw, int64_t *ba) {
    *bw = r.dw ? ceil_div((int64_t)32 * r.Op * r.Ip, kSumCols) : 0;
    *ba = r.da ? ceil_div((int64_t)32 * r.Ap, kSumCols) : 0;
    const int64_t bb = r.db ? ceil_div((int64_t)32 * r.Bp, kSumCols) : 0;
    return *bw + *ba + bb;
}

// Column sums of the partial arrays P[S][N] (each partial row contiguous):
// thread (column, phase) sums rows phase, phase + 16, ... in order, then
// phase 0 adds the 16 phase sums in order; then the 1/32, the output
// mapping (padded columns dropped) and the STE mask.
__global__ __launch_bounds__(kSumCols * kSumPhases) void hadamard_bwd_reduce_kernel(BwdSum r) {
    __shared__ double part[kSumPhases][kSumCols];
    int64_t bw, ba;
    sum_blocks(r, &bw, &ba);
    int64_t blk = blockIdx.x;
    int kind;  // 0 dW, 1 dalpha, 2 dbeta
    const float *P;
    int64_t N;
    int S;
    if (blk < bw) {
        kind = 0, P = r.pw, N = (int64_t)32 * r.Op * r.Ip, S = r.Sw;
    } else if ((blk -= bw) < ba) {
        kind = 1, P = r.pa, N = (int64_t)32 * r.Ap, S = r.Sa;
    } else {
        blk -= ba;
        kind = 2, P = r.pb, N = (int64_t)32 * r.Bp, S = r.Sb;
    }
    const int cx = threadIdx.x % kSumCols, ph = threadIdx.x / kSumCols;
    const int64_t n = blk * kSumCols + cx;
    double acc = 0.0;
    if (n < N)
        for (int s = ph; s < S; s += kSumPhases) acc += (double)P[(int64_t)s * N + n];
    part[ph][cx] = acc;
    __syncthreads();
    if (ph != 0 || n >= N) return;
    double tot = 0.0;
#pragma unroll
    for (int p = 0; p < kSumPhases; ++p) tot += part[p][cx];
    const float v = (float)(tot * 0.03125);
    if (kind == 0) {
        const int i = (int)(n % r.Ip);
        const int64_t go = n / r.Ip;
        const int o = (int)(go % r.Op), g = (int)(go / r.Op);
        if (o >= r.out_o || i >= r.in_o) return;
        const int64_t f = ((int64_t)g * r.out_o + o) * r.in_o + i;
        float out = v;
        if (r.latent) {
            const float w = r.latent[f];
            out = (w >= -1.5f && w <= 1.5f) ? v : 0.f;
        }
        r.dw[f] = out;
    } else if (kind == 1) {
        const int i = (int)(n % r.Ap), g = (int)(n / r.Ap);
        if (i < r.in_o) r.da[g * r.in_o + i] = v;
    } else {
        const int o = (int)(n % r.Bp), g = (int)(n / r.Bp);
        if (o < r.out_o) r.db[g * r.out_o + o] = v;
    }
}

// ---------------------------------------------------------------- planning

struct BwdChunk {
    int Sa, tpa;  // red pass for dx / dalpha: splits, tiles per split
    int Sb, tpb;  // red pass for dbeta
    int Sw, tpw;  // dW pass: workgroups per (nt, c), tiles per workgroup
};

static int split_count(int n_tiles, int per_split_min, int64_t target, int *tps) {
    int64_t S = target < 1 ? 1 : target;
    const int64_t maxS = ceil_div(n_tiles, per_split_min);
    if (S > maxS) S = maxS;
    if (S < 1) S = 1;
    *tps = (int)ceil_div(n_tiles, S);
    return (int)ceil_div(n_tiles, *tps);
}

static BwdChunk plan_chunk(int64_t rows, int in_o, int out_o) {
    const int n_tiles = (int)ceil_div(rows, kTile);
    const int Nt = (int)ceil_div(out_o, kNTile), Kc = (int)ceil_div(in_o, kKChunk);
    const int64_t waves = (int64_t)device_info().cu_count;  // per red role
    BwdChunk p;
    p.Sa = split_count(n_tiles, 1, ceil_div(waves, Kc), &p.tpa);  // transposed layer: Kc output tiles
    p.Sb = split_count(n_tiles, 1, ceil_div(waves, Nt), &p.tpb);
    p.Sw = split_count(n_tiles, kWaves, ceil_div((int64_t)device_info().cu_count / 2, (int64_t)Nt * Kc), &p.tpw);
    return p;
}

struct BwdLayout {
    int64_t rows_max;
    int64_t Sa, Sb, Sw;                 // total partial rows over all chunks
    int64_t off_b, off_w, bytes;        // byte offsets of the dbeta / dW partials, total
};

static BwdLayout plan(int64_t M, int64_t in_o, int64_t out_o, int64_t ld, int64_t esz) {
    BwdLayout L{};
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * esz);
    rows_max = rows_max / kTile * kTile;
    if (rows_max < kTile) {
        L.rows_max = 0;
        return L;
    }
    L.rows_max = balanced_rows(M, rows_max, kTile);
    for (int64_t r0 = 0; r0 < M; r0 += L.rows_max) {
        const int64_t rows = (M - r0) < L.rows_max ? (M - r0) : L.rows_max;
        const BwdChunk p = plan_chunk(rows, (int)in_o, (int)out_o);
        L.Sa += p.Sa;
        L.Sb += p.Sb;
        L.Sw += p.Sw;
    }
    const int64_t Ap = ceil_div(in_o, kNTile) * kNTile, Bp = ceil_div(out_o, kNTile) * kNTile;
    const int64_t bytes_a = L.Sa * 32 * Ap * 4, bytes_b = L.Sb * 32 * Bp * 4, bytes_w = L.Sw * 32 * Bp * Ap * 4;
    L.off_b = ceil_div(bytes_a, 256) * 256;
    L.off_w = L.off_b + ceil_div(bytes_b, 256) * 256;
    L.bytes = L.off_w + bytes_w;
    return L;
}

}  // namespace walsh

using namespace walsh;

WALSH_EXPORT int walsh_hadamard_pack_transpose(const uint8_t *packed, int64_t in_o, int64_t out_o, uint8_t *packed_t,
                                               void *stream) {
    if (!packed || !packed_t) return set_error(WALSH_EINVAL, "walsh_hadamard_pack_transpose: null pointer");
    if (in_o <= 0 || out_o <= 0 || in_o > (1 << 20) || out_o > (1 << 20))
        return set_error(WALSH_EINVAL, "walsh_hadamard_pack_transpose: bad shape in_o=%lld out_o=%lld",
                         (long long)in_o, (long long)out_o);
    const int64_t total = 32 * in_o * ceil_div(out_o, 4);
    int grid = (int)ceil_div(total, 256);
    if (grid > 4096) grid = 4096;
    launch(hadamard_pack_transpose_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, packed, (int)in_o,
           (int)out_o, packed_t);
    return check_hip(hipGetLastError(), "walsh_hadamard_pack_transpose launch");
}

WALSH_EXPORT int64_t walsh_hadamard_bwd_workspace_bytes(int64_t M, int64_t in_o, int64_t out_o, int dtype) {
    if (M <= 0 || in_o <= 0 || out_o <= 0 || in_o > 65536 || out_o > 65536) return 0;
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4;
    const int64_t ld = 32 * (in_o > out_o ? in_o : out_o);
    return plan(M, in_o, out_o, ld, esz).bytes;
}

WALSH_EXPORT int walsh_hadamard_linear_ex_bwd(const void *x, int64_t ldx, int64_t gsx, const void *gy, int64_t ldg,
                                              int64_t gsy, int64_t M, int64_t in_o, int64_t out_o,
                                              const uint8_t *kweight, const uint8_t *kweight_t, const float *alpha,
                                              const float *beta, const float *latent, void *gx, int64_t ldgx,
                                              float *dalpha, float *dbeta, float *dweight, int dtype, void *workspace,
                                              int64_t workspace_bytes, void *stream) {
    const char *fn = "walsh_hadamard_linear_ex_bwd";
    if ((M > 0 && (!x || !gy)) || !alpha || !beta) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || in_o <= 0 || out_o <= 0 || in_o > 65536 || out_o > 65536)
        return set_error(WALSH_EINVAL, "%s: bad shape M=%lld in_o=%lld out_o=%lld", fn, (long long)M,
                         (long long)in_o, (long long)out_o);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d not supported", fn, dtype);
    if (gsx < in_o || gsy < out_o || ldx < 32 * gsx || ldg < 32 * gsy || (gx && ldgx < 32 * gsx))
        return set_error(WALSH_EINVAL, "%s: strides too small (ldx=%lld gsx=%lld ldg=%lld gsy=%lld ldgx=%lld)", fn,
                         (long long)ldx, (long long)gsx, (long long)ldg, (long long)gsy, (long long)ldgx);
    const bool need_a = gx || dalpha, need_b = dbeta != nullptr, need_w = dweight != nullptr;
    if (need_a && !kweight_t) return set_error(WALSH_EINVAL, "%s: dx / dalpha need kweight_t", fn);
    if (need_b && !kweight) return set_error(WALSH_EINVAL, "%s: dbeta needs kweight", fn);
    const bool bf16 = dtype == WALSH_BF16;
    const int64_t esz = bf16 ? 2 : 4;
    int64_t ld = ldx > ldg ? ldx : ldg;
    if (gx && ldgx > ld) ld = ldgx;
    // the workspace query assumes dense rows; strided rows may need more chunks
    const BwdLayout L = plan(M, in_o, out_o, ld, esz);
    if (M > 0 && L.rows_max == 0) return set_error(WALSH_ENOTSUP, "%s: row stride too large", fn);
    if (M > 0 && (!workspace || workspace_bytes < L.bytes))
        return set_error(WALSH_EINVAL, "%s: workspace of %lld bytes < %lld needed", fn, (long long)workspace_bytes,
                         (long long)L.bytes);
    hipStream_t s = (hipStream_t)stream;
    const int Nt = (int)ceil_div(out_o, kNTile), Kc = (int)ceil_div(in_o, kKChunk);
    const int Ap = Kc * kKChunk, Bp = Nt * kNTile;
    float *pa = (float *)workspace;
    float *pb = (float *)((char *)workspace + L.off_b);
    float *pw = (float *)((char *)workspace + L.off_w);
    const size_t valign = bf16 ? 8 : 16;
    const int64_t maxlds = device_info().max_shared_per_block;
    auto lut = [&](void) { return (size_t)(bf16 ? lut_bytes<true>() : lut_bytes<false>()); };

    int64_t ia = 0, ib = 0, iw = 0;  // partial rows written so far
    const size_t lds_red = lut() + (size_t)16 * 128 * (Nt + Kc);
    const size_t lds_dw = (size_t)16 * 128 * (Nt + Kc) + (size_t)32 * 64 * 16;
    const size_t lds = need_w && lds_dw > lds_red ? lds_dw : lds_red;
    if ((int64_t)lds > maxlds) return set_error(WALSH_ENOTSUP, "%s: shape needs %zu B of LDS", fn, lds);
    for (int64_t r0 = 0; r0 < M; r0 += L.rows_max) {
        const int64_t rows = (M - r0) < L.rows_max ? (M - r0) : L.rows_max;
        const BwdChunk p = plan_chunk(rows, (int)in_o, (int)out_o);
        const char *xc = (const char *)x + r0 * ldx * esz;
        const char *gc = (const char *)gy + r0 * ldg * esz;
        char *gxc = gx ? (char *)gx + r0 * ldgx * esz : nullptr;
        BwdJob j{};
        auto base = [&](HadArgs &h) {
            h.M = (int)rows;
            h.kw3 = nullptr;
            h.tpb = 0;
            h.bstride = 0;
            h.xspan = 0;
            h.rope = nullptr;
            h.rope_T = 1;
            h.rope_D = 4;
            h.rope_row0 = 0;
        };
        // transposed layer on gy: in' = out_o, out' = in_o, alpha' = beta,
        // beta' = alpha (stores dx), aux = x (dalpha)
        base(j.a);
        j.a.x = gc; j.a.ldx = ldg; j.a.in_o = (int)out_o; j.a.out_o = (int)in_o; j.a.Nt = Kc; j.a.Kc = Nt;
        j.a.gsx = (int)gsy; j.a.gsy = (int)gsx; j.a.kw = kweight_t; j.a.alpha = beta; j.a.beta = alpha;
        j.a.beta_h = (int)in_o; j.a.y = gxc; j.a.ldy = gx ? ldgx : 0;
        j.ra = BwdRed{xc, ldx, (int)gsx, pa + ia * 32 * Ap, p.Sa, p.tpa};
        j.nA = need_a ? (int)ceil_div((int64_t)p.Sa * Kc, kWaves) : 0;
        // the layer on x without beta or store, aux = gy (dbeta)
        base(j.b);
        j.b.x = xc; j.b.ldx = ldx; j.b.in_o = (int)in_o; j.b.out_o = (int)out_o; j.b.Nt = Nt; j.b.Kc = Kc;
        j.b.gsx = (int)gsx; j.b.gsy = (int)gsy; j.b.kw = kweight; j.b.alpha = alpha; j.b.beta = nullptr;
        j.b.beta_h = 0; j.b.y = nullptr; j.b.ldy = 0;
        j.rb = BwdRed{gc, ldg, (int)gsy, pb + ib * 32 * Bp, p.Sb, p.tpb};
        j.nB = need_b ? (int)ceil_div((int64_t)p.Sb * Nt, kWaves) : 0;
        // x and gy as transform inputs (dW)
        base(j.wx);
        j.wx.x = xc; j.wx.ldx = ldx; j.wx.in_o = (int)in_o; j.wx.Kc = Kc; j.wx.gsx = (int)gsx; j.wx.alpha = alpha;
        base(j.wg);
        j.wg.x = gc; j.wg.ldx = ldg; j.wg.in_o = (int)out_o; j.wg.Kc = Nt; j.wg.gsx = (int)gsy; j.wg.alpha = beta;
        j.dw = BwdDW{pw + iw * 32 * (int64_t)Bp * Ap, p.Sw, p.tpw};
        j.nW = need_w ? p.Sw * Nt * Kc : 0;
        const bool vec = gsy % 4 == 0 && gsx % 4 == 0 && ldx % 4 == 0 && ldg % 4 == 0 &&
                         (!gx || ldgx % 4 == 0) && (uintptr_t)gc % valign == 0 && (uintptr_t)xc % valign == 0 &&
                         (!gx || (uintptr_t)gxc % valign == 0);
        const dim3 G((unsigned)(j.nW + j.nA + j.nB)), B(kThreads);
#define WALSH_BWD(T, MMA, V, ST) launch((hadamard_bwd_kernel<T, MMA, V, ST>), G, B, lds, s, j)
        if (bf16) {
            if (vec) { if (gx) WALSH_BWD(uint16_t, true, true, true); else WALSH_BWD(uint16_t, true, true, false); }
            else     { if (gx) WALSH_BWD(uint16_t, true, false, true); else WALSH_BWD(uint16_t, true, false, false); }
        } else {
            if (vec) { if (gx) WALSH_BWD(float, false, true, true); else WALSH_BWD(float, false, true, false); }
            else     { if (gx) WALSH_BWD(float, false, false, true); else WALSH_BWD(float, false, false, false); }
        }
#undef WALSH_BWD
        const int rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
        if (need_a) ia += p.Sa;
        if (need_b) ib += p.Sb;
        if (need_w) iw += p.Sw;
    }
    // with M == 0 every sum is empty: the reduction writes zeros
    BwdSum r{};
    r.pa = pa; r.pb = pb; r.pw = pw;
    r.Sa = (int)ia; r.Ap = Ap; r.Sb = (int)ib; r.Bp = Bp; r.Sw = (int)iw; r.Op = Bp; r.Ip = Ap;
    r.in_o = (int)in_o; r.out_o = (int)out_o; r.latent = latent;
    r.da = dalpha; r.db = dbeta; r.dw = dweight;
    int64_t bw, ba;
    const int64_t nblk = sum_blocks(r, &bw, &ba);
    if (nblk > 0) launch(hadamard_bwd_reduce_kernel, dim3((unsigned)nblk), dim3(kSumCols * kSumPhases), 0, s, r);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_hadamard_linear_bwd(const void *x, int64_t ldx, const void *gy, int64_t ldg, int64_t M,
                                           int64_t in_o, int64_t out_o, const uint8_t *kweight,
                                           const uint8_t *kweight_t, const float *alpha, const float *beta,
                                           const float *latent, void *gx, int64_t ldgx, float *dalpha, float *dbeta,
                                           float *dweight, int dtype, void *workspace, int64_t workspace_bytes,
                                           void *stream) {
    return walsh_hadamard_linear_ex_bwd(x, ldx, in_o, gy, ldg, out_o, M, in_o, out_o, kweight, kweight_t, alpha, beta,
                                        latent, gx, ldgx, dalpha, dbeta, dweight, dtype, workspace, workspace_bytes,
                                        stream);
}
