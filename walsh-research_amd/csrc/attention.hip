// Decode attention: one new query per (sequence, head) against a KV cache of
// L positions -- what CausalSelfAttention.forward does once a cache is in use
// and T == 1 (src/model/chassis.py:441-478 with the cache of :262-330):
//     o = softmax(q . K^T / sqrt(D)) V      (no mask: every cached key counts)
//
// Split-K ("flash decoding").  The L keys of a (sequence, head) are cut into
// S chunks; workgroup (chunk, head, sequence) streams its chunk of K once to
// score it (scores kept in LDS), then its chunk of V once to accumulate
// p_j v_j with p_j = exp(score_j - chunk max), and writes (acc[D], max, sum)
// as a partial.  A combine kernel rescales the S partials to the global max
// and divides by the global sum.  D/8 lanes share a key row, each reading 16
// contiguous bytes (bf16) of it, so a wavefront reads 64/(D/8) whole rows per
// load instruction.  The cache is read exactly once: the kernel is HBM-bound.
#include <mutex>

#include "common.h"

namespace walsh {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kDecMaxChunk = 2048;  // keys per workgroup (scores in LDS)

struct DecArgs {
    const void *q;
    int64_t q_bs, q_hs;             // q[b][h][d] at b*q_bs + h*q_hs + d
    const void *k, *v;
    int64_t kv_bs, kv_hs, kv_rs;    // cache element (b, h, j, d) at b*kv_bs + h*kv_hs + j*kv_rs + d
    int L, chunk, S;
    float scale;
    float *part;                    // [B][H][S][D + 2]: acc[0..D), max, sum
};

// Sum over the LPK lanes that share a key row (aligned groups of LPK lanes).
template <int LPK>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = LPK / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// A lane's 8 elements of one cache row, loaded raw (converted at use).
template <typename T> struct Raw8;
template <> struct Raw8<uint16_t> {
    uint4 u;
    __device__ __forceinline__ void load(const uint16_t *p) { u = *(const uint4 *)p; }
    __device__ __forceinline__ void get(float (&f)[8]) const {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
};
template <> struct Raw8<float> {
    f32x4 a, b;
    __device__ __forceinline__ void load(const float *p) {
        a = *(const f32x4 *)p;
        b = *(const f32x4 *)(p + 4);
    }
    __device__ __forceinline__ void get(float (&f)[8]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[i] = a[i];
            f[4 + i] = b[i];
        }
    }
};

// One (sequence, head, chunk of keys): the chunk's scores into LDS, their
// maximum, then p = exp(score - max) and sum_j p_j v_j over the lane's rows.
// A workgroup step covers KPB keys (LPK lanes per key row); the rows are
// requested kDecGroup steps at a time, the next group while the current one
// is used, and the first group of V with the first group of K, so that V's
// first round trip overlaps the scores.  Keys past the chunk load its first
// row (finite values, never used).
constexpr int kDecGroup = 4;
template <typename T, int D>
__global__ __launch_bounds__(kDecThreads) void decode_attn_partial_kernel(DecArgs a) {
    constexpr int LPK = D / 8;             // lanes per key row
    constexpr int KPW = 64 / LPK;          // keys per wavefront step
    constexpr int KPB = KPW * kDecWaves;   // keys per workgroup step
    constexpr int G = kDecGroup;
    __shared__ float sc[kDecMaxChunk];
    __shared__ float red[kDecWaves];
    __shared__ float accl[kDecWaves][D];

    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int sub = lane % LPK, kw = lane / LPK;
    const int j0 = s * a.chunk;
    const int j1 = j0 + a.chunk < a.L ? j0 + a.chunk : a.L;
    const int n = j1 - j0;  // >= 1 by construction of S
    const int nst = (n + KPB - 1) / KPB;   // workgroup steps
    const int koff = wave * KPW + kw;      // the lane's key within a step

    const T *kb = (const T *)a.k + b * a.kv_bs + h * a.kv_hs + 8 * sub;
    const T *vb = (const T *)a.v + b * a.kv_bs + h * a.kv_hs + 8 * sub;
    auto row = [&](const T *base, int step) {
        const int jj = step * KPB + koff;
        return base + (int64_t)(j0 + (jj < n ? jj : 0)) * a.kv_rs;
    };
    Raw8<T> kc[G], kn[G], vc[G], vn[G];
#pragma unroll
    for (int i = 0; i < G; ++i) kc[i].load(row(kb, i));
#pragma unroll
    for (int i = 0; i < G; ++i) vc[i].load(row(vb, i));
    float qv[8];
    {
        Raw8<T> qr;
        qr.load((const T *)a.q + b * a.q_bs + h * a.q_hs + 8 * sub);
        qr.get(qv);
    }

    // scores of the chunk
    float mx = -INFINITY;
    for (int g0 = 0; g0 < nst; g0 += G) {
        if (g0 + G < nst) {
#pragma unroll
            for (int i = 0; i < G; ++i) kn[i].load(row(kb, g0 + G + i));
        }
#pragma unroll
        for (int i = 0; i < G; ++i) {
            if (g0 + i >= nst) break;   // workgroup-uniform
            const int jj = (g0 + i) * KPB + koff;
            float kv[8];
            kc[i].get(kv);
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d += qv[e] * kv[e];
            d = group_sum<LPK>(d) * a.scale;
            if (jj < n) {
                if (sub == 0) sc[jj] = d;
                mx = fmaxf(mx, d);
            }
        }
#pragma unroll
        for (int i = 0; i < G; ++i) kc[i] = kn[i];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < kDecWaves; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();  // red is reused for the sum

    // p_j = exp(score_j - max); acc = sum_j p_j v_j over this lane's rows
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float sum = 0.f;
    for (int g0 = 0; g0 < nst; g0 += G) {
        if (g0 + G < nst) {
#pragma unroll
            for (int i = 0; i < G; ++i) vn[i].load(row(vb, g0 + G + i));
        }
#pragma unroll
        for (int i = 0; i < G; ++i) {
            if (g0 + i >= nst) break;
            const int jj = (g0 + i) * KPB + koff;
            if (jj < n) {
                const float p = expf(sc[jj] - mx);
                float vv[8];
                vc[i].get(vv);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] += p * vv[e];
                if (sub == 0) sum += p;
            }
        }
#pragma unroll
        for (int i = 0; i < G; ++i) vc[i] = vn[i];
    }
    // reduce over the KPW row groups of the wavefront (lane bits above LPK)
#pragma unroll
    for (int off = 32; off >= LPK; off >>= 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += __shfl_xor(acc[i], off, 64);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (kw == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) accl[wave][8 * sub + i] = acc[i];
    }
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    float *dst = a.part + (((int64_t)b * gridDim.y + h) * a.S + s) * (D + 2);
    for (int d = tid; d < D; d += kDecThreads) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) t += accl[w][d];
        dst[d] = t;
    }
    if (tid == 0) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) t += red[w];
        dst[D] = mx;
        dst[D + 1] = t;
    }
}

// o[b][h][d] = sum_s acc_s[d] e^(m_s - M) / sum_s l_s e^(m_s - M), M = max_s m_s.
template <typename T, int D>
__global__ __launch_bounds__(D) void decode_attn_combine_kernel(const float *__restrict__ part, int S, int H,
                                                                void *o, int64_t o_bs, int64_t o_hs) {
    const int bh = blockIdx.x, d = threadIdx.x;
    const int b = bh / H, h = bh % H;
    const float *p = part + (int64_t)bh * S * (D + 2);
    float M = -INFINITY;
#pragma unroll 16
    for (int s = 0; s < S; ++s) M = fmaxf(M, p[s * (D + 2) + D]);
    float num = 0.f, den = 0.f;
#pragma unroll 16
    for (int s = 0; s < S; ++s) {
        const float w = expf(p[s * (D + 2) + D] - M);
        num += w * p[s * (D + 2) + d];
        den += w * p[s * (D + 2) + D + 1];
    }
    Act<T>::store((T *)o + b * o_bs + h * o_hs + d, num / den);
}

static int dec_split(int64_t L, int64_t BH, int *chunk) {
    // about 8 workgroups per CU, chunks of 128 .. kDecMaxChunk keys (measured
    // at L 4095, 32 heads: batch 1 takes 32 chunks of 128 keys, batch 16
    // four of 1024, batch 64 two of 2048)
    const int64_t want = (int64_t)device_info().cu_count * 8;
    int64_t S = ceil_div(want, BH);
    const int64_t maxS = ceil_div(L, 128);
    if (S > maxS) S = maxS;
    if (S < ceil_div(L, kDecMaxChunk)) S = ceil_div(L, kDecMaxChunk);
    if (S < 1) S = 1;
    *chunk = (int)ceil_div(L, S);
    return (int)ceil_div(L, *chunk);
}

// ---------------------------------------------------------------- causal prefill
// softmax(q k^T / sqrt(D) + causal mask) v for T queries against the same T
// keys per (sequence, head): CausalSelfAttention.forward without a cache
// (chassis.py:465, F.scaled_dot_product_attention(..., is_causal=True)).
//
// Flash-style, bf16 on 16x16x16 matrix cores.  A workgroup takes 64 queries
// (16 per wave) of one (sequence, head) and walks the keys up to its last
// query in chunks staged in LDS (K row-major, V transposed).  Each
// wave computes S^T = K Q^T, so a lane holds 4 keys of ONE query (query =
// lane % 16): the running max / sum of a query live in its 4 lanes and the
// probabilities are already the B operand of O^T = V^T P^T, whose output a
// lane again holds for its own query, as it does the row sums (a product of
// a ones matrix with P^T on the matrix core).  The row max per 64 keys takes
// two lane swaps.  Keys are staged 256 (D = 16) to 64 (D >= 64) at
// a time, the next chunk's loads in flight while the current one is used.
// Scores are float32; the probabilities are rounded to bf16 for the
// products with V and with ones (the normalisation uses the weights that
// are applied), as the reference's bf16 SDPA rounds them.  The softmax
// is VALU-bound at small head_dim (one exponential per score).
constexpr int kPfQ = 64;   // queries per workgroup

struct PfArgs {
    const uint16_t *q, *k, *v;
    uint16_t *o;
    int64_t q_sb, q_sh, q_st;        // element (b, h, t, d) at b*sb + h*sh + t*st + d
    int64_t kv_sb, kv_sh, kv_st;
    int64_t o_sb, o_sh, o_st;
    int T, nqt;
    float sl2;                       // scale * log2(e)
};

// max(a, b) as med3(a, b, +inf): the same value, without the operand
// canonicalisation the compiler puts in front of fmaxf on matrix-core
// results (no NaNs arise here: scores are finite or -inf).  +inf comes from
// a register the compiler cannot see into, or it folds med3 back into fmaxf.
__device__ __forceinline__ float opaque_inf() {
    float v;
    asm volatile("v_mov_b32 %0, 0x7f800000" : "=v"(v));
    return v;
}
__device__ __forceinline__ float max2(float a, float b, float pinf) { return __builtin_amdgcn_fmed3f(a, b, pinf); }

// max over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (a query's lanes) with
// the gfx950 row / half swaps (VALU; no LDS traffic as ds_bpermute has):
// permlane16_swap exchanges odd rows of one operand with even rows of the
// other, permlane32_swap the upper half of one with the lower half of the
// other, so with both operands equal each pair of results covers the pair.
__device__ __forceinline__ float max_over_rows(float v, float pinf) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = max2(__uint_as_float(a.x), __uint_as_float(a.y), pinf);
    const u2 b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return max2(__uint_as_float(b.x), __uint_as_float(b.y), pinf);
}

struct AttnState {
    f32x4 acc[8];      // O^T tiles (D / 16 used)
    f32x4 lacc;        // every entry: this lane's query's sum of p
    float m_run;
};

// The matrix-core fragments of one 64-key step: K rows (A of S^T = K Q^T)
// and V^T rows (A of O^T = V^T P^T), per 16-key block j and 16-wide d block c.
template <int D> struct StepFrags {
    u32x2 k[4][D / 16], v[4][D / 16];
};

// K rows kl[key * ks + d], V transposed vt[d * vs + key] (LDS); LDS row r0
// is the step's first key.
template <int D>
__device__ __forceinline__ void load_frags(StepFrags<D> &f, const uint16_t *kl, int ks, const uint16_t *vt, int vs,
                                           int r0, int n, int kq) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            f.k[j][c] = *(const u32x2 *)(kl + (r0 + 16 * j + n) * ks + 16 * c + 4 * kq);
            f.v[j][c] = *(const u32x2 *)(vt + (16 * c + n) * vs + r0 + 16 * j + 4 * kq);
        }
}

// One 64-key step of the online softmax for a wave's 16 queries, keys
// k0 .. k0 + 63.  FULL: every key of the step is at or before the wave's
// first query (no mask); otherwise keys past each query are masked and
// 16-key blocks wholly after the wave's last query are skipped.
template <int D, bool FULL>
__device__ __forceinline__ void attn_step_frags(AttnState &st, const u32x2 (&qf)[D / 16], const StepFrags<D> &f,
                                                int k0, int qw, int qi, int kq, float sl2) {
    constexpr int ND = D / 16;
    const u32x2 ones = {0x3f803f80u, 0x3f803f80u};   // four bf16 1.0
    f32x4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int kb = k0 + 16 * j;
        if (!FULL && kb > qw + 15) {           // wave-uniform
            s[j] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            continue;
        }
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < ND; ++c)
            t = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, f.k[j][c]),
                                                         __builtin_bit_cast(i16x4, qf[c]), t, 0, 0, 0);
        // t[i]: S[query qi][key kb + 4kq + i], unscaled (the scale is folded
        // into the exponent; scale > 0 keeps the max)
        if (!FULL && kb + 15 > qw) {           // the diagonal block: mask keys past the query
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (kb + 4 * kq + i > qi) t[i] = -INFINITY;
        }
        s[j] = t;
    }
    const float pinf = opaque_inf();
    // the running max is the same in a query's four lanes, so it can start
    // the chain: 16 scores and m_run in 8 three-input maxima (v_max3_f32;
    // m_run is already canonical, so the compiler puts no canonicalising
    // max in front), then the two lane swaps
    float mx = fmaxf(fmaxf(st.m_run, s[0].x), s[0].y);
    mx = fmaxf(fmaxf(mx, s[0].z), s[0].w);
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        mx = fmaxf(fmaxf(mx, s[j].x), s[j].y);
        mx = fmaxf(fmaxf(mx, s[j].z), s[j].w);
    }
    const float m_new = max_over_rows(mx, pinf);
    // v_exp_f32 directly: arguments are <= 0 (or -inf -> 0); results below
    // the float32 normal range flush to zero
    const float alpha = __builtin_amdgcn_exp2f((st.m_run - m_new) * sl2);
    st.m_run = m_new;
    const float moff = -m_new * sl2;
    u32x2 pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pv[i] = __builtin_amdgcn_exp2f(fmaf(s[j][i], sl2, moff));
        pf[j] = u32x2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
    }
    st.lacc *= alpha;
#pragma unroll
    for (int c = 0; c < ND; ++c) st.acc[c] *= alpha;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (!FULL && k0 + 16 * j > qw + 15) continue;
        // row sums of the (bf16) probabilities on the matrix core:
        // ones(16 x 16 keys) P^T puts sum_k P[query][k] in every row
        st.lacc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, ones),
                                                           __builtin_bit_cast(i16x4, pf[j]), st.lacc, 0, 0, 0);
#pragma unroll
        for (int c = 0; c < ND; ++c)
            st.acc[c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, f.v[j][c]),
                                                                 __builtin_bit_cast(i16x4, pf[j]), st.acc[c], 0, 0, 0);
    }
}

// The step with its fragments read from LDS rows r0 .. r0 + 63.
template <int D, bool FULL>
__device__ __forceinline__ void attn_step(AttnState &st, const u32x2 (&qf)[D / 16], const uint16_t *kl, int ks,
                                          const uint16_t *vt, int vs, int r0, int k0, int qw, int qi, int n, int kq,
                                          float sl2) {
    StepFrags<D> f;
    load_frags<D>(f, kl, ks, vt, vs, r0, n, kq);
    attn_step_frags<D, FULL>(st, qf, f, k0, qw, qi, kq, sl2);
}

template <int D>
__device__ __forceinline__ void attn_store(const AttnState &st, uint16_t *op, int kq) {
    const float inv = 1.0f / st.lacc[0];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        // acc[c][i]: O[query][d = 16c + 4kq + i]
        const f32x4 r = st.acc[c] * inv;
        *(u32x2 *)(op + 16 * c + 4 * kq) = u32x2{pack_bf16x2(r.x, r.y), pack_bf16x2(r.z, r.w)};
    }
}

// Keys per LDS chunk: as many as keep the tile near 20 KB, so a chunk's
// global loads are few round trips per workgroup.
template <int D> struct PfKC { static constexpr int value = D == 16 ? 256 : D == 32 ? 128 : 64; };

template <int D>
__global__ __launch_bounds__(256) void prefill_attn_kernel(PfArgs a) {
    constexpr int ND = D / 16;
    constexpr int KC = PfKC<D>::value;
    constexpr int KS = D + 4;                        // padded K row (bank spread)
    constexpr int VS = KC + 4;                       // padded row of the transposed V tile
    constexpr int PIECES = KC * D / 8;               // 16-byte pieces per tensor per chunk
    constexpr int PPT = (2 * PIECES + 255) / 256;    // pieces per thread
    __shared__ __align__(16) uint16_t k_l[KC * KS];
    __shared__ __align__(16) uint16_t vt_l[D * VS];
    const int qt = a.nqt - 1 - (int)blockIdx.x;      // longest query tiles first
    const int h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, kq = lane >> 4;
    const int qw = qt * kPfQ + wave * 16;            // this wave's first query
    const int qi = qw + n;                           // this lane's query
    const int qc = qi < a.T ? qi : a.T - 1;
    const int kend = (qt + 1) * kPfQ;                // keys this workgroup can need

    u32x2 qf[ND];
    {
        const uint16_t *qp = a.q + b * a.q_sb + h * a.q_sh + (int64_t)qc * a.q_st;
#pragma unroll
        for (int c = 0; c < ND; ++c) qf[c] = *(const u32x2 *)(qp + 16 * c + 4 * kq);
    }
    AttnState st;
#pragma unroll
    for (int c = 0; c < ND; ++c) st.acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.lacc = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m_run = -INFINITY;

    const uint16_t *kbase = a.k + b * a.kv_sb + h * a.kv_sh;
    const uint16_t *vbase = a.v + b * a.kv_sb + h * a.kv_sh;
    uint4 stg[PPT];
    // keys at or past kend are neither loaded nor read; keys past T are
    // loaded from row T - 1 (finite values that the causal mask zeroes)
    auto gload = [&](int ch) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int p = tid + 256 * i;
            const int tensor = p >= PIECES, pp = p - tensor * PIECES;
            const int key = pp / (D / 8), part = pp - key * (D / 8);
            int kidx = ch * KC + key;
            if (p < 2 * PIECES && kidx < kend) {
                kidx = kidx < a.T ? kidx : a.T - 1;
                stg[i] = *(const uint4 *)((tensor ? vbase : kbase) + (int64_t)kidx * a.kv_st + part * 8);
            }
        }
    };
    auto lstore = [&](int ch) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int p = tid + 256 * i;
            const int tensor = p >= PIECES, pp = p - tensor * PIECES;
            const int key = pp / (D / 8), part = pp - key * (D / 8);
            if (p < 2 * PIECES && ch * KC + key < kend) {
                if (!tensor) {
                    u32x2 *d = (u32x2 *)(k_l + key * KS + part * 8);
                    d[0] = u32x2{stg[i].x, stg[i].y};
                    d[1] = u32x2{stg[i].z, stg[i].w};
                } else {
                    const uint32_t w[4] = {stg[i].x, stg[i].y, stg[i].z, stg[i].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        vt_l[(part * 8 + 2 * e) * VS + key] = (uint16_t)(w[e] & 0xffffu);
                        vt_l[(part * 8 + 2 * e + 1) * VS + key] = (uint16_t)(w[e] >> 16);
                    }
                }
            }
        }
    };

    const int nch = (kend + KC - 1) / KC;
    gload(0);
    for (int ch = 0; ch < nch; ++ch) {
        __syncthreads();       // the previous chunk's readers are done
        lstore(ch);
        __syncthreads();
        if (ch + 1 < nch) gload(ch + 1);   // next chunk in flight during this one
        // 64-key steps.  Steps wholly at or before this wave's first query
        // (all but the last one or two) take the unmasked path; the step
        // holding the diagonal masks keys past each query and skips 16-key
        // blocks wholly after the wave's last query.
#pragma unroll 1
        for (int sb = 0; sb < KC / 64; ++sb) {
            const int k0 = ch * KC + sb * 64;
            if (k0 > qw + 15) break;                   // wave-uniform
            if (k0 + 63 <= qw) attn_step<D, true>(st, qf, k_l, KS, vt_l, VS, sb * 64, k0, qw, qi, n, kq, a.sl2);
            else attn_step<D, false>(st, qf, k_l, KS, vt_l, VS, sb * 64, k0, qw, qi, n, kq, a.sl2);
        }
    }
    if (qi < a.T) attn_store<D>(st, a.o + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_st, kq);
}

// head_dim 128: 128 queries per workgroup (8 waves of 16), 64-key chunks of
// K (row-major, three buffers, loaded straight into LDS two chunks ahead) and
// V (transposed through registers into two buffers, one chunk ahead) in LDS;
// one barrier per chunk.  Products on 16x16x32 bf16 MFMA: S^T = K Q^T takes 4 per 16-key
// block (a lane's A operand is 8 dims of one key, read from a K row, its B
// operand 8 dims of its query, held in registers); O^T = V^T P^T takes one
// per 16 dims and 32 keys, with the 32 keys of a product in the order the
// score accumulators hold them (slots 0-3: keys 4kq..4kq+3 of the first
// 16-key block, slots 4-7: of the second), so the probabilities are the B
// operand as computed and the V^T operand is read in the same order (one
// 16-byte read from a V^T row).  The row sums of P ride along as a product
// with a ones matrix.  Softmax, masking and roundings as prefill_attn_kernel.
constexpr int kFaQ = 128, kFaKC = 64;
// LDS: three K buffers (64 keys x 256 bytes; 16-byte chunk c of key row r at
// position c ^ (r & 15)) and two V^T buffers (128 dims x 128 bytes; chunk u
// of dim row d at position u ^ ((d >> 1) & 7)): 80 KB, two workgroups per CU.
// The swizzles keep the fragment reads (16 rows of one chunk column) and the
// V^T stores on distinct banks without padding.
constexpr int kFaKBuf = kFaKC * 256, kFaVBuf = 128 * kFaKC * 2;
constexpr int kFaLds = 3 * kFaKBuf + 2 * kFaVBuf;

// Column of key offset o (0..31) within its 32-key half of a V^T row: the
// keys of product slots 8kq .. 8kq + 7 (4kq .. 4kq + 3, then 16 + 4kq ..
// 16 + 4kq + 3) lie at 8kq .. 8kq + 7.  Keys 2m and 2m + 1 stay adjacent.
__device__ __forceinline__ int fa_vt_pos(int o) { return 8 * ((o & 15) >> 2) + 4 * (o >> 4) + (o & 3); }

__device__ __forceinline__ f32x4 fa_mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}

// One 64-key step for a wave's 16 queries (keys k0 .. k0 + 63 at LDS rows
// 0..63 of the chunk).  FULL: every key at or before the wave's first query.
template <bool FULL>
__device__ __forceinline__ void fa_step(AttnState &st, const u32x4 (&qf)[4], const uint16_t *kl, const uint16_t *vt,
                                        int k0, int qw, int qi, int n, int kq, float sl2) {
    f32x4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int kb = k0 + 16 * j;
        if (!FULL && kb > qw + 15) {           // wave-uniform
            s[j] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            continue;
        }
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
        const unsigned char *kr = (const unsigned char *)kl + (16 * j + n) * 256;
#pragma unroll
        for (int c = 0; c < 4; ++c) t = fa_mma(*(const u32x4 *)(kr + (((4 * c + kq) ^ n) << 4)), qf[c], t);
        // t[i]: S[query qi][key kb + 4kq + i], unscaled
        if (!FULL && kb + 15 > qw) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (kb + 4 * kq + i > qi) t[i] = -INFINITY;
        }
        s[j] = t;
    }
    const float pinf = opaque_inf();
    float mx = fmaxf(fmaxf(st.m_run, s[0].x), s[0].y);
    mx = fmaxf(fmaxf(mx, s[0].z), s[0].w);
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        mx = fmaxf(fmaxf(mx, s[j].x), s[j].y);
        mx = fmaxf(fmaxf(mx, s[j].z), s[j].w);
    }
    const float m_new = max_over_rows(mx, pinf);
    const float alpha = __builtin_amdgcn_exp2f((st.m_run - m_new) * sl2);
    st.m_run = m_new;
    const float moff = -m_new * sl2;
    u32x2 pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pv[i] = __builtin_amdgcn_exp2f(fmaf(s[j][i], sl2, moff));
        pf[j] = u32x2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
    }
    st.lacc *= alpha;
#pragma unroll
    for (int c = 0; c < 8; ++c) st.acc[c] *= alpha;
    const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};   // eight bf16 1.0
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (!FULL && k0 + 32 * h > qw + 15) continue;   // both 16-key blocks past the wave's queries
        const u32x4 pb = {pf[2 * h].x, pf[2 * h].y, pf[2 * h + 1].x, pf[2 * h + 1].y};
        st.lacc = fa_mma(ones, pb, st.lacc);
        // V^T rows hold each 32-key half in product order (fa_vt_pos), so a
        // lane's 8 keys are one 16-byte read (chunk 4h + kq of dim row 16c + n)
        const unsigned char *vr = (const unsigned char *)vt + n * 128 + (((4 * h + kq) ^ (n >> 1)) << 4);
#pragma unroll
        for (int c = 0; c < 8; ++c) st.acc[c] = fa_mma(*(const u32x4 *)(vr + 16 * c * 128), pb, st.acc[c]);
    }
}

__global__ __launch_bounds__(512, 2) void prefill_fa128_kernel(PfArgs a) {
    extern __shared__ __align__(1024) unsigned char fa_smem[];
    // Work items to XCDs: workgroups go to the 8 XCDs in turn (linear id w
    // on XCD w % 8), so with the query tiles on x every head's tiles would
    // land on 8 different XCDs and each L2 would fetch the head's K and V
    // again.  Instead slot s = w / 8 of XCD w % 8 takes query tile s % nqt
    // (longest first) of head group s / nqt: all tiles of one (sequence,
    // head) run on one XCD and share its L2.
    int qt, h, b;
    {
        const int H = (int)gridDim.y, BH = H * (int)gridDim.z;
        const int w = (int)blockIdx.x + a.nqt * ((int)blockIdx.y + H * (int)blockIdx.z);
        if (BH % 8 == 0) {
            const int slot = w >> 3, bh = (slot / a.nqt) * 8 + (w & 7);
            qt = a.nqt - 1 - slot % a.nqt;
            h = bh % H;
            b = bh / H;
        } else {
            qt = a.nqt - 1 - (int)blockIdx.x;
            h = blockIdx.y;
            b = blockIdx.z;
        }
    }
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, kq = lane >> 4;
    const int qw = qt * kFaQ + wave * 16;            // this wave's first query
    const int qi = qw + n;                           // this lane's query
    const int qc = qi < a.T ? qi : a.T - 1;
    const int kend = min((qt + 1) * kFaQ, ((a.T + kFaKC - 1) / kFaKC) * kFaKC);  // keys the workgroup can need
    u32x4 qf[4];
    {
        const uint16_t *qp = a.q + b * a.q_sb + h * a.q_sh + (int64_t)qc * a.q_st;
#pragma unroll
        for (int c = 0; c < 4; ++c) qf[c] = *(const u32x4 *)(qp + 32 * c + 8 * kq);
    }
    AttnState st;
#pragma unroll
    for (int c = 0; c < 8; ++c) st.acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.lacc = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m_run = -INFINITY;
    const uint16_t *kbase = a.k + b * a.kv_sb + h * a.kv_sh;
    const uint16_t *vbase = a.v + b * a.kv_sb + h * a.kv_sh;
    // K: straight to LDS (buffer loads into LDS, no registers): wave w fills
    // key rows 8w .. 8w + 7 of a chunk, 4 rows (1 KB) per instruction, lane l
    // landing at position l % 16 of row 8w + 4i + l / 16, which holds chunk
    // (l % 16) ^ (row & 15).  Keys past T load row T - 1 (finite values the
    // causal mask zeroes).
    // byte span of one head's K (or V) rows; below 4 GiB (the host checks)
    const uint32_t kspan = (uint32_t)(((int64_t)(a.T - 1) * a.kv_st + 128) * 2);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(kbase, kspan);
    auto kload = [&](int ch) {
        // the LDS destination of a buffer-to-LDS load is wave-uniform (M0)
        unsigned char *dst = fa_smem + (ch % 3) * kFaKBuf + __builtin_amdgcn_readfirstlane(wave) * 2048;
        int t = tid;
        asm volatile("" : "+v"(t));
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = 8 * (t >> 6) + 4 * i + (t & 63) / 16;
            int kk = ch * kFaKC + row;
            kk = kk < a.T ? kk : a.T - 1;
            const uint32_t off = (uint32_t)kk * (uint32_t)(2 * a.kv_st) + 16 * ((t % 16) ^ (row & 15));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (__attribute__((address_space(3))) void *)(dst + i * 1024),
                                                     16, off, 0, 0, 0);
        }
    };
    // V: through registers (two chunks ahead in two sets), then to V^T as
    // 32-bit pairs of keys: thread tid takes keys 2 (tid % 32), + 1 at dims
    // 8 (tid / 32) ..; lanes 32..63 of a wave write the row pair's other
    // member first, so each store instruction covers both bank halves
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vbase, kspan);
    auto vload = [&](int ch, u32x4 (&vr)[2]) {
        int t = tid;
        asm volatile("" : "+v"(t));
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            int kv = ch * kFaKC + 2 * (t % 32) + u;
            kv = kv < a.T ? kv : a.T - 1;
            vr[u] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (uint32_t)kv * (uint32_t)(2 * a.kv_st) + 16 * (t / 32),
                                                          0, 0);
        }
    };
    auto vstore = [&](int ch, const u32x4 (&vr)[2]) {
        unsigned char *vt = fa_smem + 3 * kFaKBuf + (ch & 1) * kFaVBuf;
        // the lane's store addresses are recomputed for every chunk (a few
        // VALU ops) rather than held in registers across the loop
        int t = tid;
        asm volatile("" : "+v"(t));
        const int key = 2 * (t % 32), d0 = 8 * (t / 32);
        const int col = (key & 32) + fa_vt_pos(key & 31), sw = (t >> 5) & 1;
        const uint32_t wa[4] = {vr[0].x, vr[0].y, vr[0].z, vr[0].w};
        const uint32_t wb[4] = {vr[1].x, vr[1].y, vr[1].z, vr[1].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // dims 2e, 2e + 1: (key, key + 1) packed low / high
            const uint32_t p0 = __builtin_amdgcn_perm(wb[e], wa[e], 0x05040100u);
            const uint32_t p1 = __builtin_amdgcn_perm(wb[e], wa[e], 0x07060302u);
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
                const int d = d0 + 2 * e + (t2 ^ sw);
                const int pos = (((col >> 3) ^ ((d >> 1) & 7)) << 3) + (col & 7);
                *(uint32_t *)(vt + d * 128 + pos * 2) = (t2 ^ sw) ? p1 : p0;
            }
        }
    };
    // Loads are issued unconditionally (past the last chunk they fetch clamped
    // rows into buffers no wave reads again), so every wave has the same
    // number of loads in flight and the waits below count exactly.  The
    // barriers are bare s_barrier: a __syncthreads would also wait for the
    // K loads of the chunk after next.
    const int nch = kend / kFaKC;
    u32x4 va[2];
    kload(0);
    vload(0, va);
    kload(1);
    vstore(0, va);
    asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)" ::: "memory");   // K(0) in LDS, V^T(0) stored
    asm volatile("s_barrier" ::: "memory");
    // chunk ch: V(ch + 1) to registers and K(ch + 2) to LDS requested, the
    // products of ch, V^T(ch + 1) stored, K(ch + 1) waited for, one barrier
    for (int ch = 0; ch < nch; ++ch) {
        vload(ch + 1, va);
        kload(ch + 2);
        const uint16_t *kl = (const uint16_t *)(fa_smem + (ch % 3) * kFaKBuf);
        const uint16_t *vt = (const uint16_t *)(fa_smem + 3 * kFaKBuf + (ch & 1) * kFaVBuf);
        const int k0 = ch * kFaKC;
        // lane-derived offsets are recomputed for every chunk rather than
        // held in registers across the loop
        int ln = lane;
        asm volatile("" : "+v"(ln));
        if (k0 <= qw + 15) {               // keys at or before some query of the wave
            if (k0 + kFaKC - 1 <= qw) fa_step<true>(st, qf, kl, vt, k0, qw, qi, ln & 15, ln >> 4, a.sl2);
            else fa_step<false>(st, qf, kl, vt, k0, qw, qi, ln & 15, ln >> 4, a.sl2);
        }
        vstore(ch + 1, va);                // the V^T buffer of chunk ch - 1
        asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)" ::: "memory");   // all but K(ch + 2)
        asm volatile("s_barrier" ::: "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // no load into LDS outlives the workgroup
    if (qi < a.T) attn_store<128>(st, a.o + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_st, kq);
}

// Whole-head variant, for heads whose K and V fit in LDS together (T_pad *
// (D + 4) * 2 + D * (T_pad + 4) * 2 bytes; head_dim 16 up to about 2,200
// positions): one workgroup of 16 waves per (sequence, head) stages K
// (row-major) and V (transposed) once, then the waves take 16-query
// sub-tiles from a counter in LDS, longest first (sub-tile s needs
// floor((16 s + 15) / 64) + 1 key steps).  A static split of equal step
// counts does not balance: the SIMD issues from its oldest wave first, so
// the oldest waves finish early and the rest run with fewer waves per SIMD
// (half the VALU rate at one).  Taking work as a wave frees up keeps every
// wave busy until the last few short sub-tiles.  No barriers after the
// staging.  (gridDim.z workgroups may share a head, each with its own
// counter over every gridDim.z-th sub-tile; one measured fastest at
// head_dim 16, T = 1024.)
constexpr int kPhWaves = 16;

template <int D>
__global__ __launch_bounds__(64 * kPhWaves) void prefill_attn_head_kernel(PfArgs a, int tpad) {
    constexpr int ND = D / 16;
    extern __shared__ __align__(16) uint16_t ph_smem[];
    // padded rows: the 16 lanes of a fragment read (one key or one d per
    // lane, 8 bytes each) start 2 dwords mod 32 apart, so they hit distinct
    // banks (K rows of D + 4 elements; V^T rows of tpad + 4, tpad % 64 == 0)
    const int ks = D + 4;
    const int vs = tpad + 4;
    uint16_t *k_l = ph_smem;                         // [tpad][ks]
    uint16_t *vt_l = ph_smem + tpad * ks;            // [D][vs]
    __shared__ int next_tile;
    // heads to XCDs: the dispatcher deals consecutive workgroups to the 8
    // XCDs in turn, so with H % 8 == 0 workgroup w runs on XCD w % 8.  Head
    // (w % 8) (H / 8) + w / 8 puts H / 8 consecutive heads on one XCD: the
    // 64 / D heads whose q / k / v share a 128-byte line of [B, T, H, D] rows
    // (four at head_dim 16) fetch it into one L2 instead of four.
    const int H = (int)gridDim.x, wg = (int)blockIdx.x;
    const int h = H % 8 == 0 ? (wg % 8) * (H / 8) + wg / 8 : wg, b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int n = lane & 15, kq = lane >> 4;
    if (tid == 0) next_tile = 0;
    const uint16_t *kbase = a.k + b * a.kv_sb + h * a.kv_sh;
    const uint16_t *vbase = a.v + b * a.kv_sb + h * a.kv_sh;
    // stage K and V^T; rows T .. tpad - 1 are zeros (finite, masked).  The
    // rows come in batches of kPhBatch per thread, every load of a batch
    // requested before its stores (buffer loads, zero past T: no branch
    // around them, so one round trip per batch rather than per row)
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(kbase, (uint32_t)(((int64_t)(a.T - 1) * a.kv_st + D) * 2));
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(vbase, (uint32_t)(((int64_t)(a.T - 1) * a.kv_st + D) * 2));
    constexpr int kPhBatch = 4;
    const int nstage = tpad * (D / 8);
    for (int p0 = tid; p0 < nstage; p0 += kPhBatch * 64 * kPhWaves) {
        uint4 kv[kPhBatch], vv[kPhBatch];
#pragma unroll
        for (int i = 0; i < kPhBatch; ++i) {
            const int p = p0 + i * 64 * kPhWaves, key = p / (D / 8), part = p - key * (D / 8);
            const uint32_t off =
                (p < nstage && key < a.T) ? (uint32_t)(((int64_t)key * a.kv_st + part * 8) * 2) : kOOB;
            kv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
            vv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < kPhBatch; ++i) {
            const int p = p0 + i * 64 * kPhWaves, key = p / (D / 8), part = p - key * (D / 8);
            if (p >= nstage) break;
            u32x2 *kd = (u32x2 *)(k_l + key * ks + part * 8);   // 8-byte aligned rows
            kd[0] = u32x2{kv[i].x, kv[i].y};
            kd[1] = u32x2{kv[i].z, kv[i].w};
            const uint32_t w[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vt_l[(part * 8 + 2 * e) * vs + key] = (uint16_t)(w[e] & 0xffffu);
                vt_l[(part * 8 + 2 * e + 1) * vs + key] = (uint16_t)(w[e] >> 16);
            }
        }
    }
    __syncthreads();
    // this workgroup's sub-tiles: nst - 1 - (z + Z j), j = 0, 1, ... (z =
    // blockIdx.z, Z = gridDim.z), in that order (decreasing length)
    const int nst = tpad / 16, Z = (int)gridDim.z, z = (int)blockIdx.z;
    for (;;) {
        int j = 0;
        if (lane == 0) j = atomicAdd(&next_tile, 1);
        j = __builtin_amdgcn_readfirstlane(__shfl(j, 0));
        const int stile = nst - 1 - (z + Z * j);
        if (stile < 0) break;  // wave-uniform: every wave leaves once the counter passes the last sub-tile
        const int qw = 16 * stile, qi = qw + n;
        const int qc = qi < a.T ? qi : a.T - 1;
        u32x2 qf[ND];
        const uint16_t *qp = a.q + b * a.q_sb + h * a.q_sh + (int64_t)qc * a.q_st;
#pragma unroll
        for (int c = 0; c < ND; ++c) qf[c] = *(const u32x2 *)(qp + 16 * c + 4 * kq);
        AttnState st;
#pragma unroll
        for (int c = 0; c < ND; ++c) st.acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        st.lacc = f32x4{0.f, 0.f, 0.f, 0.f};
        st.m_run = -INFINITY;
        // each step's fragments are read from LDS one step ahead, into two
        // sets used in turn (two steps per trip)
        const int last = qw + 15;
        StepFrags<D> f0, f1;
        load_frags<D>(f0, k_l, ks, vt_l, vs, 0, n, kq);
        auto step = [&](const StepFrags<D> &f, int k0) {
            if (k0 + 63 <= qw) attn_step_frags<D, true>(st, qf, f, k0, qw, qi, kq, a.sl2);
            else attn_step_frags<D, false>(st, qf, f, k0, qw, qi, kq, a.sl2);
        };
#pragma unroll 1
        for (int k0 = 0; k0 <= last; k0 += 128) {
            if (k0 + 64 <= last) load_frags<D>(f1, k_l, ks, vt_l, vs, k0 + 64, n, kq);
            step(f0, k0);
            if (k0 + 64 > last) break;
            if (k0 + 128 <= last) load_frags<D>(f0, k_l, ks, vt_l, vs, k0 + 128, n, kq);
            step(f1, k0 + 64);
        }
        if (qi < a.T) attn_store<D>(st, a.o + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_st, kq);
    }
}

}  // namespace walsh

using namespace walsh;

WALSH_EXPORT int64_t walsh_decode_attention_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t D) {
    if (B <= 0 || H <= 0 || L <= 0 || D <= 0) return 0;
    int chunk;
    const int S = dec_split(L, B * H, &chunk);
    return B * H * S * (D + 2) * (int64_t)sizeof(float);
}

// The checks and the two launches of a decode attention call, with the
// split-K partials at ``part`` (B * H * S * (D + 2) floats, every slot written
// by the partial kernel before the combine reads it).
static int decode_attention_run(const char *fn, const void *q, int64_t q_bs, int64_t q_hs, const void *k,
                                const void *v, int64_t kv_bs, int64_t kv_hs, int64_t kv_rs, int64_t B, int64_t H,
                                int64_t L, int64_t D, float scale, void *o, int64_t o_bs, int64_t o_hs, int dtype,
                                float *part, int64_t part_bytes, bool static_part, void *stream) {
    if (B < 0 || H <= 0 || L <= 0 || B > 65535 || H > 65535 || L > (1 << 30))
        return set_error(WALSH_EINVAL, "%s: bad shape B=%lld H=%lld L=%lld", fn, (long long)B, (long long)H,
                         (long long)L);
    if (D != 16 && D != 32 && D != 64 && D != 128)
        return set_error(WALSH_ENOTSUP, "%s: head_dim %lld (16, 32, 64 or 128)", fn, (long long)D);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d", fn, dtype);
    if (B == 0) return WALSH_OK;
    if (!q || !k || !v || !o || !part) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    const int64_t vec = 8;
    if (q_bs % vec || q_hs % vec || kv_bs % vec || kv_hs % vec || kv_rs % vec || kv_rs < D ||
        (uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16)
        return set_error(WALSH_ENOTSUP, "%s: q / cache rows must be 16-byte aligned with strides multiple of 8", fn);
    int chunk;
    const int S = dec_split(L, B * H, &chunk);
    const int64_t need = B * H * S * (D + 2) * (int64_t)sizeof(float);
    if (part_bytes < need) {
        if (static_part)
            return set_error(WALSH_ENOTSUP, "%s: B=%lld H=%lld L=%lld D=%lld need %lld bytes of split-K scratch, above "
                             "the static maximum of %lld (use walsh_decode_attention with a workspace)", fn,
                             (long long)B, (long long)H, (long long)L, (long long)D, (long long)need,
                             (long long)part_bytes);
        return set_error(WALSH_EINVAL, "%s: workspace too small", fn);
    }
    DecArgs a{q, q_bs, q_hs, k, v, kv_bs, kv_hs, kv_rs, (int)L, chunk, S, scale, part};
    hipStream_t s = (hipStream_t)stream;
    const dim3 G((unsigned)S, (unsigned)H, (unsigned)B);
#define WALSH_DEC(T, DD)                                                                                          \
    do {                                                                                                          \
        launch(decode_attn_partial_kernel<T, DD>, G, dim3(kDecThreads), 0, s, a);                                 \
        launch(decode_attn_combine_kernel<T, DD>, dim3((unsigned)(B * H)), dim3(DD), 0, s, (const float *)part,     \
               S, (int)H, o, o_bs, o_hs);                                                                         \
    } while (0)
    if (dtype == WALSH_BF16) {
        if (D == 128) WALSH_DEC(uint16_t, 128);
        else if (D == 64) WALSH_DEC(uint16_t, 64);
        else if (D == 32) WALSH_DEC(uint16_t, 32);
        else WALSH_DEC(uint16_t, 16);
    } else {
        if (D == 128) WALSH_DEC(float, 128);
        else if (D == 64) WALSH_DEC(float, 64);
        else if (D == 32) WALSH_DEC(float, 32);
        else WALSH_DEC(float, 16);
    }
#undef WALSH_DEC
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_decode_attention(const void *q, int64_t q_bs, int64_t q_hs, const void *k, const void *v,
                                        int64_t kv_bs, int64_t kv_hs, int64_t kv_rs, int64_t B, int64_t H, int64_t L,
                                        int64_t D, float scale, void *o, int64_t o_bs, int64_t o_hs, int dtype,
                                        void *workspace, int64_t workspace_bytes, void *stream) {
    return decode_attention_run("walsh_decode_attention", q, q_bs, q_hs, k, v, kv_bs, kv_hs, kv_rs, B, H, L, D, scale,
                                o, o_bs, o_hs, dtype, (float *)workspace, workspace_bytes, false, stream);
}

// ---------------------------------------------------------------- allocation-free decode attention
// walsh_decode_attention_static keeps the split-K partials in this file-scope
// device array instead of a caller workspace, for callers that cannot
// allocate.  Each GPU the library runs on holds its own copy until the
// process ends; every call on one GPU shares it, so calls that overlap on one
// GPU (other streams, other host threads) race on it.  Host code never passes
// the array's name to a kernel: its device address comes from
// hipGetSymbolAddress, looked up once per device on the first call there.
constexpr int64_t kDecScratchBytes = 8ll << 20;
constexpr int kScratchMaxDevices = 64;
static __device__ __align__(256) float scratch[kDecScratchBytes / sizeof(float)];

static int dec_scratch(const char *fn, float **out) {
    static std::mutex mu;
    static float *ptrs[kScratchMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return check_hip(e, fn);
    if (dev < 0 || dev >= kScratchMaxDevices)
        return set_error(WALSH_ENOTSUP, "%s: device %d beyond the %d this build tracks", fn, dev, kScratchMaxDevices);
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return check_hip(e, fn);
        if (!p) return set_error(WALSH_EHIP, "%s: no device address for the scratch array", fn);
        ptrs[dev] = (float *)p;
    }
    *out = ptrs[dev];
    return WALSH_OK;
}

WALSH_EXPORT int walsh_decode_attention_static(const void *q, int64_t q_bs, int64_t q_hs, const void *k, const void *v,
                                               int64_t kv_bs, int64_t kv_hs, int64_t kv_rs, int64_t B, int64_t H,
                                               int64_t L, int64_t D, float scale, void *o, int64_t o_bs, int64_t o_hs,
                                               int dtype, void *stream) {
    const char *fn = "walsh_decode_attention_static";
    float *part = nullptr;
    const int rc = dec_scratch(fn, &part);
    if (rc) return rc;
    return decode_attention_run(fn, q, q_bs, q_hs, k, v, kv_bs, kv_hs, kv_rs, B, H, L, D, scale, o, o_bs, o_hs, dtype,
                                part, kDecScratchBytes, true, stream);
}

WALSH_EXPORT int walsh_prefill_attention(const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void *k,
                                         const void *v, int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t B,
                                         int64_t H, int64_t T, int64_t D, float scale, void *o, int64_t o_sb,
                                         int64_t o_sh, int64_t o_st, int dtype, void *stream) {
    const char *fn = "walsh_prefill_attention";
    if (B < 0 || H <= 0 || T < 0 || B > 65535 || H > 65535 || T > (1 << 24))
        return set_error(WALSH_EINVAL, "%s: bad shape B=%lld H=%lld T=%lld", fn, (long long)B, (long long)H,
                         (long long)T);
    if (D != 16 && D != 32 && D != 64 && D != 128)
        return set_error(WALSH_ENOTSUP, "%s: head_dim %lld (16, 32, 64 or 128)", fn, (long long)D);
    if (dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d (bf16 only)", fn, dtype);
    if (B == 0 || T == 0) return WALSH_OK;
    if (!q || !k || !v || !o) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    const int64_t st[9] = {q_sb, q_sh, q_st, kv_sb, kv_sh, kv_st, o_sb, o_sh, o_st};
    for (int i = 0; i < 9; ++i)
        if (st[i] % 8 || st[i] < 0)
            return set_error(WALSH_ENOTSUP, "%s: strides must be non-negative multiples of 8 elements", fn);
    if ((uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16 || (uintptr_t)o % 16)
        return set_error(WALSH_ENOTSUP, "%s: q, k, v, o must be 16-byte aligned", fn);
    PfArgs a{(const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)v, (uint16_t *)o, q_sb, q_sh, q_st,
             kv_sb, kv_sh, kv_st, o_sb, o_sh, o_st, (int)T, (int)ceil_div(T, kPfQ), scale * 1.4426950408889634f};
    hipStream_t s = (hipStream_t)stream;
    // whole heads in LDS when they fit (tpad rows of K and of V^T, padded;
    // 256 bytes kept for the kernel's static LDS, its sub-tile counter)
    const int64_t tpad = ceil_div(T, 64) * 64;
    const int64_t head_lds = (tpad * (D + 4) + D * (tpad + 4)) * 2;
    if (D == 16 && head_lds + 256 <= device_info().max_shared_per_block) {
        launch(prefill_attn_head_kernel<16>, dim3((unsigned)H, (unsigned)B, 1u), dim3(64 * kPhWaves),
               (uint32_t)head_lds, s, a, (int)tpad);
        return check_hip(hipGetLastError(), fn);
    }
    // prefill_fa128_kernel addresses a head's K and V rows with 32-bit byte offsets
    const bool fa_span_ok = ((T - 1) * kv_st + 128) * 2 <= (int64_t)UINT32_MAX;
    if (D == 128 && fa_span_ok && (size_t)kFaLds <= (size_t)device_info().max_shared_per_block) {
        PfArgs a2 = a;
        a2.nqt = (int)ceil_div(T, kFaQ);
        launch(prefill_fa128_kernel, dim3((unsigned)a2.nqt, (unsigned)H, (unsigned)B), dim3(512),
               (uint32_t)kFaLds, s, a2);
        return check_hip(hipGetLastError(), fn);
    }
    const dim3 G((unsigned)a.nqt, (unsigned)H, (unsigned)B);
    if (D == 16) launch(prefill_attn_kernel<16>, G, dim3(256), 0, s, a);
    else if (D == 32) launch(prefill_attn_kernel<32>, G, dim3(256), 0, s, a);
    else if (D == 64) launch(prefill_attn_kernel<64>, G, dim3(256), 0, s, a);
    else launch(prefill_attn_kernel<128>, G, dim3(256), 0, s, a);
    return check_hip(hipGetLastError(), fn);
}
