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

template <typename T> struct Ld8;
template <> struct Ld8<uint16_t> {
    static __device__ __forceinline__ void load(const uint16_t *p, float (&f)[8]) {
        const uint4 u = *(const uint4 *)p;
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
};
template <> struct Ld8<float> {
    static __device__ __forceinline__ void load(const float *p, float (&f)[8]) {
        const f32x4 a = *(const f32x4 *)p, b = *(const f32x4 *)(p + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[i] = a[i];
            f[4 + i] = b[i];
        }
    }
};

// Sum over the LPK lanes that share a key row (aligned groups of LPK lanes).
template <int LPK>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = LPK / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <typename T, int D>
__global__ __launch_bounds__(kDecThreads) void decode_attn_partial_kernel(DecArgs a) {
    constexpr int LPK = D / 8;             // lanes per key row
    constexpr int KPW = 64 / LPK;          // keys per wavefront step
    constexpr int KPB = KPW * kDecWaves;   // keys per workgroup step
    __shared__ float sc[kDecMaxChunk];
    __shared__ float red[kDecWaves];
    __shared__ float accl[kDecWaves][D];

    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int sub = lane % LPK, kw = lane / LPK;
    const int j0 = s * a.chunk;
    const int j1 = j0 + a.chunk < a.L ? j0 + a.chunk : a.L;
    const int n = j1 - j0;  // >= 1 by construction of S

    float qv[8];
    Ld8<T>::load((const T *)a.q + b * a.q_bs + h * a.q_hs + 8 * sub, qv);
    const T *kb = (const T *)a.k + b * a.kv_bs + h * a.kv_hs + 8 * sub;
    const T *vb = (const T *)a.v + b * a.kv_bs + h * a.kv_hs + 8 * sub;

    // scores of the chunk (rows past j1 are not read)
    float mx = -INFINITY;
    for (int base = 0; base < n; base += KPB) {
        const int jj = base + wave * KPW + kw;
        float d = 0.f;
        if (jj < n) {
            float kv[8];
            Ld8<T>::load(kb + (int64_t)(j0 + jj) * a.kv_rs, kv);
#pragma unroll
            for (int i = 0; i < 8; ++i) d += qv[i] * kv[i];
        }
        d = group_sum<LPK>(d) * a.scale;
        if (jj < n) {
            if (sub == 0) sc[jj] = d;
            mx = fmaxf(mx, d);
        }
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
    for (int base = 0; base < n; base += KPB) {
        const int jj = base + wave * KPW + kw;
        if (jj < n) {
            const float p = expf(sc[jj] - mx);
            float vv[8];
            Ld8<T>::load(vb + (int64_t)(j0 + jj) * a.kv_rs, vv);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] += p * vv[i];
            if (sub == 0) sum += p;
        }
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
    for (int s = 0; s < S; ++s) M = fmaxf(M, p[s * (D + 2) + D]);
    float num = 0.f, den = 0.f;
    for (int s = 0; s < S; ++s) {
        const float w = expf(p[s * (D + 2) + D] - M);
        num += w * p[s * (D + 2) + d];
        den += w * p[s * (D + 2) + D + 1];
    }
    Act<T>::store((T *)o + b * o_bs + h * o_hs + d, num / den);
}

static int dec_split(int64_t L, int64_t BH, int *chunk) {
    // enough workgroups to cover the chip twice, chunks of 128 .. kDecMaxChunk keys
    const int64_t want = (int64_t)device_info().cu_count * 2;
    int64_t S = ceil_div(want, BH);
    const int64_t maxS = ceil_div(L, 128);
    if (S > maxS) S = maxS;
    if (S < ceil_div(L, kDecMaxChunk)) S = ceil_div(L, kDecMaxChunk);
    if (S < 1) S = 1;
    *chunk = (int)ceil_div(L, S);
    return (int)ceil_div(L, *chunk);
}

}  // namespace walsh

using namespace walsh;

WALSH_EXPORT int64_t walsh_decode_attention_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t D) {
    if (B <= 0 || H <= 0 || L <= 0 || D <= 0) return 0;
    int chunk;
    const int S = dec_split(L, B * H, &chunk);
    return B * H * S * (D + 2) * (int64_t)sizeof(float);
}

WALSH_EXPORT int walsh_decode_attention(const void *q, int64_t q_bs, int64_t q_hs, const void *k, const void *v,
                                        int64_t kv_bs, int64_t kv_hs, int64_t kv_rs, int64_t B, int64_t H, int64_t L,
                                        int64_t D, float scale, void *o, int64_t o_bs, int64_t o_hs, int dtype,
                                        void *workspace, int64_t workspace_bytes, void *stream) {
    const char *fn = "walsh_decode_attention";
    if (B < 0 || H <= 0 || L <= 0 || B > 65535 || H > 65535 || L > (1 << 30))
        return set_error(WALSH_EINVAL, "%s: bad shape B=%lld H=%lld L=%lld", fn, (long long)B, (long long)H,
                         (long long)L);
    if (D != 16 && D != 32 && D != 64 && D != 128)
        return set_error(WALSH_ENOTSUP, "%s: head_dim %lld (16, 32, 64 or 128)", fn, (long long)D);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d", fn, dtype);
    if (B == 0) return WALSH_OK;
    if (!q || !k || !v || !o || !workspace) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    const int64_t vec = 8;
    if (q_bs % vec || q_hs % vec || kv_bs % vec || kv_hs % vec || kv_rs % vec || kv_rs < D ||
        (uintptr_t)q % 16 || (uintptr_t)k % 16 || (uintptr_t)v % 16)
        return set_error(WALSH_ENOTSUP, "%s: q / cache rows must be 16-byte aligned with strides multiple of 8", fn);
    int chunk;
    const int S = dec_split(L, B * H, &chunk);
    if (workspace_bytes < B * H * S * (D + 2) * (int64_t)sizeof(float))
        return set_error(WALSH_EINVAL, "%s: workspace too small", fn);
    DecArgs a{q, q_bs, q_hs, k, v, kv_bs, kv_hs, kv_rs, (int)L, chunk, S, scale, (float *)workspace};
    hipStream_t s = (hipStream_t)stream;
    const dim3 G((unsigned)S, (unsigned)H, (unsigned)B);
#define WALSH_DEC(T, DD)                                                                                          \
    do {                                                                                                          \
        launch(decode_attn_partial_kernel<T, DD>, G, dim3(kDecThreads), 0, s, a);                                 \
        launch(decode_attn_combine_kernel<T, DD>, dim3((unsigned)(B * H)), dim3(DD), 0, s, (const float *)workspace, \
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
