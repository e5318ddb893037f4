// Absmean ternary quantisation and the 2-bit packed code format.
//
// gamma = mean(|W|) + 1e-8 over a whole tensor (src/model/physics.py:24),
// codes = clamp(round_half_even(W / gamma), -1, 1) (physics.py:27-29),
// packed byte = v0<<6 | v1<<4 | v2<<2 | v3 with v = code + 1
// (src/model/fht_cuda.py:65-93).
#include "common.h"

namespace walsh {

constexpr int kGammaThreads = 1024;

// One workgroup; fixed element->thread assignment and a fixed-shape tree, so
// the float64 sum (and the float32 gamma) is identical on every run.
__global__ __launch_bounds__(kGammaThreads) void gamma_kernel(const float *__restrict__ w, int64_t n,
                                                              float *__restrict__ gamma) {
    __shared__ double part[kGammaThreads];
    const int t = threadIdx.x;
    double acc = 0.0;
    const bool vec = ((uintptr_t)w & 15) == 0;
    int64_t head = 0;
    if (vec) {
        const int64_t n4 = n / 4;
        const f32x4 *w4 = (const f32x4 *)w;
        for (int64_t i = t; i < n4; i += kGammaThreads) {
            f32x4 v = w4[i];
            acc += (double)fabsf(v.x);
            acc += (double)fabsf(v.y);
            acc += (double)fabsf(v.z);
            acc += (double)fabsf(v.w);
        }
        head = n4 * 4;
    }
    for (int64_t i = head + t; i < n; i += kGammaThreads) acc += (double)fabsf(w[i]);
    part[t] = acc;
    __syncthreads();
    for (int s = kGammaThreads / 2; s > 0; s >>= 1) {
        if (t < s) part[t] += part[t + s];
        __syncthreads();
    }
    if (t == 0) {
        const float mean = (float)(part[0] / (double)n);
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
