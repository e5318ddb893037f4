// Absmean ternary quantisation and the 2-bit packed code format.
//
// gamma = mean(|W|) + 1e-8 over a whole tensor (src/model/physics.py:24),
// codes = clamp(round_half_even(W / gamma), -1, 1) (physics.py:27-29),
// packed byte = v0<<6 | v1<<4 | v2<<2 | v3 with v = code + 1
// (src/model/fht_cuda.py:65-93).
#include "common.h"

namespace walsh {

constexpr int kGammaThreads = 1024;

// Error-free sum of two doubles (Knuth's TwoSum): s + e == a + b exactly.
__device__ inline void two_sum(double a, double b, double &s, double &e) {
    s = a + b;
    const double z = s - a;
    e = (a - (s - z)) + (b - z);
}

// One workgroup; fixed element->thread assignment and a fixed-shape tree, so
// the result is identical on every run.  The sum of |w| is carried as a
// double-double (hi + lo, TwoSum at every addition), about 100 bits, so the
// float32 mean is the correctly rounded mean of the exact sum (the division
// keeps the remainder through an fma) -- a value that does not depend on the
// reduction order, unlike a float32 or plain float64 sum.
__global__ __launch_bounds__(kGammaThreads) void gamma_kernel(const float *__restrict__ w, int64_t n,
                                                              float *__restrict__ gamma) {
    __shared__ double part_hi[kGammaThreads];
    __shared__ double part_lo[kGammaThreads];
    const int t = threadIdx.x;
    double hi = 0.0, lo = 0.0;
    auto add = [&](float v) {
        double e;
        two_sum(hi, (double)fabsf(v), hi, e);
        lo += e;
    };
    const bool vec = ((uintptr_t)w & 15) == 0;
    int64_t head = 0;
    if (vec) {
        const int64_t n4 = n / 4;
        const f32x4 *w4 = (const f32x4 *)w;
        for (int64_t i = t; i < n4; i += kGammaThreads) {
            f32x4 v = w4[i];
            add(v.x);
            add(v.y);
            add(v.z);
            add(v.w);
        }
        head = n4 * 4;
    }
    for (int64_t i = head + t; i < n; i += kGammaThreads) add(w[i]);
    part_hi[t] = hi;
    part_lo[t] = lo;
    __syncthreads();
    for (int s = kGammaThreads / 2; s > 0; s >>= 1) {
        if (t < s) {
            double h, e;
            two_sum(part_hi[t], part_hi[t + s], h, e);
            part_lo[t] = part_lo[t] + part_lo[t + s] + e;
            part_hi[t] = h;
        }
        __syncthreads();
    }
    if (t == 0) {
        const double nd = (double)n, h = part_hi[0], l = part_lo[0];
        double q = h / nd;
        const double r = fma(-q, nd, h);  // h - q*n exactly
        q += (r + l) / nd;
        const float mean = (float)q;
        gamma[0] = mean + 1e-8f;
    }
}

__global__ void quantize_kernel(const float *__restrict__ w, int64_t rows, int64_t K,
                                const float *__restrict__ gamma, int8_t *__restrict__ codes,
                                uint8_t *__restrict__ packed, float *__restrict__ scaled) {
    const int64_t kp4 = ceil_div(K, 4);
    const int64_t total = rows * kp4;
    const float g = gamma[0];
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total;
         b += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = b / kp4;
        const int64_t k0 = (b - r * kp4) * 4;
        uint32_t byte = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t k = k0 + j;
            int c = 0;
            if (k < K) {
                const float wv = w[r * K + k];
                float q = rintf(__fdiv_rn(wv, g));
                q = fminf(fmaxf(q, -1.0f), 1.0f);
                c = (int)q;
                if (codes) codes[r * K + k] = (int8_t)c;
                if (scaled) scaled[r * K + k] = (float)c * g;
            }
            byte |= (uint32_t)(c + 1) << (6 - 2 * j);
        }
        if (packed) packed[b] = (uint8_t)byte;
    }
}

__global__ void unpack_kernel(const uint8_t *__restrict__ packed, int64_t rows, int64_t K,
                              int8_t *__restrict__ codes) {
    const int64_t kp4 = ceil_div(K, 4);
    const int64_t total = rows * K;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / K;
        const int64_t k = e - r * K;
        const uint32_t byte = packed[r * kp4 + k / 4];
        codes[e] = (int8_t)((int)((byte >> (6 - 2 * (k & 3))) & 3u) - 1);
    }
}

static int grid_for(int64_t work, int block) {
    const int64_t cap = (int64_t)device_info().cu_count * 16;
    int64_t g = ceil_div(work, block);
    if (g > cap) g = cap;
    return (int)(g < 1 ? 1 : g);
}

// ---------------------------------------------------------------- .walsh v4 bitmask + sign
// A ternary tensor of `total` values stored as a bitmask (bit p of the
// little-endian bit stream: value p is non-zero) and a sign stream (bit r:
// the r-th non-zero is +1 when set, -1 when clear) (compress.py:36-93,
// generate_compressed.py:70-105).  The value at position p is therefore
// sign[rank(p)] with rank(p) = the number of set mask bits before p, a prefix
// popcount.  Three passes over 32-bit mask words: per-word counts with a
// workgroup exclusive scan, a scan of the workgroup sums, then the decode,
// one output byte (4 codes of the 2-bit packed layout) per thread.
constexpr int kMaskWordsPerBlock = 256;

__device__ __forceinline__ uint32_t mask_word(const uint8_t *__restrict__ m, int64_t nb, int64_t w) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t b = 4 * w + i;
        if (b < nb) v |= (uint32_t)m[b] << (8 * i);
    }
    return v;
}

__global__ __launch_bounds__(kMaskWordsPerBlock) void bitmask_count_kernel(const uint8_t *__restrict__ mask, int64_t nb,
                                                                           int64_t nwords, int64_t total,
                                                                           uint32_t *__restrict__ word_pref,
                                                                           uint32_t *__restrict__ block_sum) {
    __shared__ uint32_t sc[kMaskWordsPerBlock];
    const int t = threadIdx.x;
    const int64_t w = (int64_t)blockIdx.x * kMaskWordsPerBlock + t;
    uint32_t c = 0;
    if (w < nwords) {
        uint32_t v = mask_word(mask, nb, w);
        const int64_t valid = total - 32 * w;  // bits past `total` are ignored
        if (valid < 32) v &= (1u << valid) - 1u;
        c = (uint32_t)__popc(v);
    }
    sc[t] = c;
    __syncthreads();
    for (int off = 1; off < kMaskWordsPerBlock; off <<= 1) {  // inclusive Hillis-Steele scan
        const uint32_t add = t >= off ? sc[t - off] : 0u;
        __syncthreads();
        sc[t] += add;
        __syncthreads();
    }
    if (w < nwords) word_pref[w] = sc[t] - c;
    if (t == kMaskWordsPerBlock - 1) block_sum[blockIdx.x] = sc[t];
}

// Exclusive scan of the workgroup sums in place, one workgroup, chunks of 1024.
__global__ __launch_bounds__(1024) void bitmask_scan_kernel(uint32_t *__restrict__ block_sum, int64_t nblk) {
    __shared__ uint32_t sc[1024];
    __shared__ uint32_t carry;
    const int t = threadIdx.x;
    if (t == 0) carry = 0;
    __syncthreads();
    for (int64_t base = 0; base < nblk; base += 1024) {
        const int64_t i = base + t;
        const uint32_t c = i < nblk ? block_sum[i] : 0u;
        sc[t] = c;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const uint32_t add = t >= off ? sc[t - off] : 0u;
            __syncthreads();
            sc[t] += add;
            __syncthreads();
        }
        if (i < nblk) block_sum[i] = carry + sc[t] - c;
        __syncthreads();
        if (t == 1023) carry += sc[1023];
        __syncthreads();
    }
}

__global__ void bitmask_decode_kernel(const uint8_t *__restrict__ mask, int64_t nb, const uint8_t *__restrict__ sign,
                                      int64_t ns, int64_t nnz, const uint32_t *__restrict__ word_pref,
                                      const uint32_t *__restrict__ block_pref, int64_t rows, int64_t K,
                                      uint8_t *__restrict__ packed, int8_t *__restrict__ codes) {
    const int64_t kp4 = ceil_div(K, 4);
    const int64_t total_b = rows * kp4;
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total_b;
         b += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = b / kp4;
        const int64_t k0 = (b - r * kp4) * 4;
        uint32_t byte = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t k = k0 + j;
            int c = 0;
            if (k < K) {
                const int64_t p = r * K + k;
                const int64_t w = p >> 5;
                const int bit = (int)(p & 31);
                const uint32_t v = mask_word(mask, nb, w);
                if ((v >> bit) & 1u) {
                    const int64_t rank = (int64_t)block_pref[w / kMaskWordsPerBlock] + word_pref[w] +
                                         __popc(v & ((1u << bit) - 1u));
                    // non-zeros past num_nonzero keep the value 0, as the reference loader does
                    if (rank < nnz && (rank >> 3) < ns) c = ((sign[rank >> 3] >> (rank & 7)) & 1u) ? 1 : -1;
                }
                if (codes) codes[p] = (int8_t)c;
            }
            byte |= (uint32_t)(c + 1) << (6 - 2 * j);
        }
        if (packed) packed[b] = (uint8_t)byte;
    }
}

// Straight-through estimators' backward, elementwise over n weights:
//   mode 0 (physics.quantize_ternary, physics.py:43-50): the value
//     w_clamped + (w_quant - w_clamped).detach() passes gradient only through
//     w.clamp(-1.5, 1.5): g_latent = g * [-1.5 <= w <= 1.5];
//   mode 1 (moe.TernaryAbsmeanSTE.backward, moe.py:289-294):
//     g_latent = clamp(g, -2, 2).
__global__ void ste_bwd_kernel(const float *__restrict__ g, const float *__restrict__ w, int64_t n, int mode,
                               float *__restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = g[i];
        float r;
        if (mode == 0) {
            const float x = w[i];
            r = (x >= -1.5f && x <= 1.5f) ? v : 0.f;
        } else {
            r = fminf(fmaxf(v, -2.f), 2.f);
            if (v != v) r = v;  // NaN passes through, as torch.clamp does
        }
        out[i] = r;
    }
}

}  // namespace walsh

using namespace walsh;

WALSH_EXPORT int walsh_ternary_ste_bwd(const float *grad, const float *w, int64_t n, int mode, float *out,
                                       void *stream) {
    if (n < 0 || (mode != 0 && mode != 1)) return set_error(WALSH_EINVAL, "walsh_ternary_ste_bwd: n=%lld mode=%d",
                                                            (long long)n, mode);
    if (n == 0) return WALSH_OK;
    if (!grad || !out || (mode == 0 && !w)) return set_error(WALSH_EINVAL, "walsh_ternary_ste_bwd: null pointer");
    const int block = 256;
    const int grid = grid_for(n, block);
    launch(ste_bwd_kernel, dim3(grid), dim3(block), 0, (hipStream_t)stream, grad, w, n, mode, out);
    return check_hip(hipGetLastError(), "walsh_ternary_ste_bwd launch");
}

WALSH_EXPORT int walsh_ternary_gamma(const float *w, int64_t n, float *gamma, void *stream) {
    if (!w || !gamma) return set_error(WALSH_EINVAL, "walsh_ternary_gamma: null pointer");
    if (n <= 0) return set_error(WALSH_EINVAL, "walsh_ternary_gamma: n must be positive (got %lld)", (long long)n);
    launch(gamma_kernel, dim3(1), dim3(kGammaThreads), 0, (hipStream_t)stream, w, n, gamma);
    return check_hip(hipGetLastError(), "walsh_ternary_gamma launch");
}

WALSH_EXPORT int walsh_ternary_quantize(const float *w, int64_t rows, int64_t K, const float *gamma,
                                        int8_t *codes, uint8_t *packed, float *scaled, void *stream) {
    if (!w || !gamma) return set_error(WALSH_EINVAL, "walsh_ternary_quantize: null input pointer");
    if (rows <= 0 || K <= 0)
        return set_error(WALSH_EINVAL, "walsh_ternary_quantize: rows and K must be positive");
    const int block = 256;
    const int grid = grid_for(rows * ceil_div(K, 4), block);
    launch(quantize_kernel, dim3(grid), dim3(block), 0, (hipStream_t)stream, w, rows, K, gamma,
                       codes, packed, scaled);
    return check_hip(hipGetLastError(), "walsh_ternary_quantize launch");
}

WALSH_EXPORT int walsh_ternary_unpack(const uint8_t *packed, int64_t rows, int64_t K, int8_t *codes,
                                      void *stream) {
    if (!packed || !codes) return set_error(WALSH_EINVAL, "walsh_ternary_unpack: null pointer");
    if (rows <= 0 || K <= 0) return set_error(WALSH_EINVAL, "walsh_ternary_unpack: rows and K must be positive");
    const int block = 256;
    const int grid = grid_for(rows * K, block);
    launch(unpack_kernel, dim3(grid), dim3(block), 0, (hipStream_t)stream, packed, rows, K, codes);
    return check_hip(hipGetLastError(), "walsh_ternary_unpack launch");
}

WALSH_EXPORT int64_t walsh_bitmask_workspace_bytes(int64_t total) {
    if (total <= 0) return 0;
    const int64_t nwords = ceil_div(total, 32), nblk = ceil_div(nwords, kMaskWordsPerBlock);
    return (nwords + nblk) * (int64_t)sizeof(uint32_t);
}

WALSH_EXPORT int walsh_ternary_from_bitmask(const uint8_t *bitmask, int64_t bitmask_bytes, const uint8_t *sign_bits,
                                            int64_t sign_bytes, int64_t num_nonzero, int64_t rows, int64_t K,
                                            uint8_t *packed, int8_t *codes, void *workspace, int64_t workspace_bytes,
                                            void *stream) {
    const char *fn = "walsh_ternary_from_bitmask";
    if (rows <= 0 || K <= 0 || bitmask_bytes < 0 || sign_bytes < 0 || num_nonzero < 0)
        return set_error(WALSH_EINVAL, "%s: bad sizes", fn);
    const int64_t total = rows * K;
    if (total >= (int64_t)1 << 32) return set_error(WALSH_ENOTSUP, "%s: more than 2^32 values", fn);
    if ((!bitmask && bitmask_bytes) || (!sign_bits && sign_bytes) || (!packed && !codes))
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    const int64_t need = walsh_bitmask_workspace_bytes(total);
    if (!workspace || workspace_bytes < need)
        return set_error(WALSH_EINVAL, "%s: workspace of %lld bytes < %lld", fn, (long long)workspace_bytes,
                         (long long)need);
    const int64_t nwords = ceil_div(total, 32), nblk = ceil_div(nwords, kMaskWordsPerBlock);
    uint32_t *word_pref = (uint32_t *)workspace;
    uint32_t *block_pref = word_pref + nwords;
    hipStream_t s = (hipStream_t)stream;
    launch(bitmask_count_kernel, dim3((unsigned)nblk), dim3(kMaskWordsPerBlock), 0, s, bitmask, bitmask_bytes, nwords,
           total, word_pref, block_pref);
    launch(bitmask_scan_kernel, dim3(1), dim3(1024), 0, s, block_pref, nblk);
    const int block = 256;
    launch(bitmask_decode_kernel, dim3(grid_for(rows * ceil_div(K, 4), block)), dim3(block), 0, s, bitmask,
           bitmask_bytes, sign_bits, sign_bytes, num_nonzero, word_pref, block_pref, rows, K, packed, codes);
    return check_hip(hipGetLastError(), fn);
}
