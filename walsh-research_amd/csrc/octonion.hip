// Octonion (Cayley-Dickson) ternary linear forward.
//
// Reference: OctonionTernaryLinearRef.forward (src/model/physics.py:66-82) and
// the fused GPU path cayley_dickson_fused_kernel
// (src/model/cayley_dickson_cuda.py:313-421):
//     y_i = beta * sum_j S[i][j] x_j @ W[i ^ j]^T      (i, j = 0..7)
// with the sign table S of src/model/constants.py:13-31.
//
// MI355X design.  The 8x8 block structure is a signed permutation of only 8
// distinct ternary blocks, so at weight-preparation time it is expanded once
// into the dense block matrix B[i*out_o + n][j*in_o + k] = S[i][j] W[i^j][n][k]
// (still exactly {-1, 0, 1}, stored bf16 or f32, K-contiguous).  The forward
// is then one matrix-core GEMM  y = (x B^T) * beta  with 128x128 output tiles,
// four wavefronts each owning 64x64 (4x4 tiles of 16x16), K staged through
// double-buffered LDS, and beta fused into the epilogue.
#include "common.h"
#include "gemm256.h"

namespace walsh {

__constant__ int8_t kOctSign[8][8] = {
    {+1, -1, -1, -1, -1, -1, -1, -1}, {+1, +1, +1, -1, +1, -1, -1, +1}, {+1, -1, +1, +1, +1, +1, -1, -1},
    {+1, +1, -1, +1, +1, -1, +1, -1}, {+1, -1, -1, -1, +1, +1, +1, +1}, {+1, +1, -1, +1, -1, +1, -1, +1},
    {+1, +1, +1, -1, -1, +1, +1, -1}, {+1, -1, +1, +1, -1, -1, +1, +1}};

constexpr int kBM = 128, kBN = 128;
constexpr int kGemmThreads = 256;

// B[i*out_o + n][j*in_o + k] = S[i][j] * code(W[i^j][n][k]), from packed
// codes [8, out_o, ceil(in_o/4)]; row length Kp (>= 8*in_o, zero padded).
template <typename T>
__global__ void octonion_expand_kernel(const uint8_t *__restrict__ packed, int in_o, int out_o, int Kp,
                                       T *__restrict__ B) {
    const int64_t N = 8LL * out_o;
    const int64_t total = N * Kp;
    const int kp4 = (int)ceil_div(in_o, 4);
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e / Kp;
        const int col = (int)(e - row * Kp);
        float v = 0.f;
        if (col < 8 * in_o) {
            const int i = (int)(row / out_o), n = (int)(row - (int64_t)i * out_o);
            const int j = col / in_o, k = col - j * in_o;
            const int w = i ^ j;
            const uint32_t byte = packed[((int64_t)w * out_o + n) * kp4 + k / 4];
            const int code = (int)((byte >> (6 - 2 * (k & 3))) & 3u) - 1;
            v = (float)(kOctSign[i][j] * code);
        }
        Act<T>::store(B + e, v);
    }
}

// -------------------------------------------------------------------- GEMM
// y[m, n] = beta[n % out_o] * sum_k x[m, k] B[n, k]
// T = uint16_t (bf16 operands, 16x16x32 bf16 MFMA) or float (16x16x4 f32 MFMA).
template <typename T> struct GemmCfg;
template <> struct GemmCfg<uint16_t> { static constexpr int BK = 32; };  // 64 B per row
template <> struct GemmCfg<float> { static constexpr int BK = 16; };     // 64 B per row
constexpr int kLdsStride = 80;  // 64 B + 16 B pad: 8 consecutive rows cover all banks once

typedef Gemm256Args OctArgs;

template <typename T>
__global__ __launch_bounds__(kGemmThreads, 2) void octonion_gemm_kernel(OctArgs a) {
    constexpr int BK = GemmCfg<T>::BK;
    constexpr uint32_t esz = sizeof(T);
    __shared__ __align__(16) unsigned char lds[2][2][kBM * kLdsStride];  // [buf][A/B]

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.x * kBM, n0 = blockIdx.y * kBN;
    // split-K: split blockIdx.z sums columns [k_lo, k_hi)
    const int split = blockIdx.z;
    const int k_lo = a.kspan > 0 ? (int)(split * a.kspan) : 0;
    const int k_hi = a.kspan > 0 ? (int)(k_lo + a.kspan < a.K ? k_lo + a.kspan : a.K) : a.K;
    const int kb_hi = a.kspan > 0 ? k_hi : a.Kp;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * esz));
    const __amdgpu_buffer_rsrc_t br = make_rsrc(a.B, (uint32_t)((int64_t)a.N * a.Kp * esz));

    // global -> register staging: a 128-row x 64-byte tile is 512 chunks of
    // 16 B; thread t moves chunks t and t + 256 of A and of B per K step
    const int ch0 = tid, ch1 = tid + kGemmThreads;  // chunk id = row*4 + part
    const int ra0 = ch0 >> 2, pa0 = ch0 & 3, ra1 = ch1 >> 2, pa1 = ch1 & 3;
    constexpr int kElemsPerChunk = 16 / esz;

    auto load_tile = [&](int k0, u32x4 (&ra)[2], u32x4 (&rb)[2]) {
        const int ka0 = k_lo + k0 + pa0 * kElemsPerChunk, ka1 = k_lo + k0 + pa1 * kElemsPerChunk;
        const int am0 = m0 + ra0, am1 = m0 + ra1;
        ra[0] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, (am0 < a.M && ka0 < k_hi) ? (uint32_t)(((int64_t)am0 * a.ldx + ka0) * esz) : kOOB, 0, 0);
        ra[1] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, (am1 < a.M && ka1 < k_hi) ? (uint32_t)(((int64_t)am1 * a.ldx + ka1) * esz) : kOOB, 0, 0);
        const int bn0 = n0 + ra0, bn1 = n0 + ra1;
        rb[0] = __builtin_amdgcn_raw_buffer_load_b128(
            br, (bn0 < a.N && ka0 < kb_hi) ? (uint32_t)(((int64_t)bn0 * a.Kp + ka0) * esz) : kOOB, 0, 0);
        rb[1] = __builtin_amdgcn_raw_buffer_load_b128(
            br, (bn1 < a.N && ka1 < kb_hi) ? (uint32_t)(((int64_t)bn1 * a.Kp + ka1) * esz) : kOOB, 0, 0);
    };
    auto store_tile = [&](int buf, const u32x4 (&ra)[2], const u32x4 (&rb)[2]) {
        *(u32x4 *)(&lds[buf][0][ra0 * kLdsStride + pa0 * 16]) = ra[0];
        *(u32x4 *)(&lds[buf][0][ra1 * kLdsStride + pa1 * 16]) = ra[1];
        *(u32x4 *)(&lds[buf][1][ra0 * kLdsStride + pa0 * 16]) = rb[0];
        *(u32x4 *)(&lds[buf][1][ra1 * kLdsStride + pa1 * 16]) = rb[1];
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = (int)ceil_div(k_hi - k_lo, BK);
    u32x4 ra[2], rb[2];
    load_tile(0, ra, rb);
    store_tile(0, ra, rb);
    __syncthreads();

    const int fr = lane & 15, fq = lane >> 4;  // fragment row, 16-byte chunk
    for (int kk = 0; kk < nk; ++kk) {
        const int cur = kk & 1;
        if (kk + 1 < nk) load_tile((kk + 1) * BK, ra, rb);
        u32x4 af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            af[i] = *(const u32x4 *)(&lds[cur][0][(wm * 64 + i * 16 + fr) * kLdsStride + fq * 16]);
            bf[i] = *(const u32x4 *)(&lds[cur][1][(wn * 64 + i * 16 + fr) * kLdsStride + fq * 16]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (sizeof(T) == 2) {
                    // A rows = tokens (i), B rows = outputs (j): D[token][out]
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[i]),
                                                                        __builtin_bit_cast(bf16x8, bf[j]), acc[i][j],
                                                                        0, 0, 0);
                } else {
                    const f32x4 av = __builtin_bit_cast(f32x4, af[i]);
                    const f32x4 bv = __builtin_bit_cast(f32x4, bf[j]);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s], bv[s], acc[i][j], 0, 0, 0);
                }
            }
        if (kk + 1 < nk) store_tile(cur ^ 1, ra, rb);
        __syncthreads();
    }

    // epilogue: lane holds D[m = 4*fq + r][n = fr] of each 16x16 tile
    const int64_t yspan = a.kspan > 0 ? (int64_t)(gridDim.z - 1) * a.ysplit + (int64_t)a.M * a.ldy
                                      : (int64_t)a.M * a.ldy;
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)(yspan * esz));
    const int64_t ybase = (int64_t)split * a.ysplit;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 64 + j * 16 + fr;
        const float b = n < a.N ? (a.beta ? a.beta[n % a.out_o] : 1.f) : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 64 + i * 16 + 4 * fq + r;
                const uint32_t off =
                    (m < a.M && n < a.N) ? (uint32_t)((ybase + (int64_t)m * a.ldy + n) * esz) : kOOB;
                Buf4<T>::store1(acc[i][j][r] * b, yr, off, 0);
            }
    }
}

// ------------------------------------------------------------------ backward
// The layer is y = (x B^T) .* beta~ with beta~[i*out_o + n] = beta[n].  For an
// output gradient gy:
//   gx = (gy .* beta~) B = gy Bt^T with Bt[j*in_o + m][i*out_o + n] =
//        S[i][j] W[i^j][n][m] beta[n]    (the forward GEMM on Bt, no beta)
//   C  = gy^T x                          [8*out_o][8*in_o], K = tokens
//   dW[w][n][m] = beta[n] sum_i S[i][i^w] C[i*out_o + n][(i^w)*in_o + m]
//   dbeta[n]    = sum_{i,j,m} S[i][j] W[i^j][n][m] C[i*out_o + n][j*in_o + m]
// (each weight block w = i^j appears once per output part i).  The STE of
// physics.quantize_ternary passes dW where -1.5 <= latent <= 1.5.

// Bt rows j*in_o + m, row length Np (>= 8*out_o, zero padded).
template <typename T>
__global__ void octonion_expand_t_kernel(const uint8_t *__restrict__ packed, int in_o, int out_o,
                                         const float *__restrict__ beta, int Np, T *__restrict__ Bt) {
    const int64_t R = 8LL * in_o;
    const int64_t total = R * Np;
    const int kp4 = (int)ceil_div(in_o, 4);
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e / Np;
        const int col = (int)(e - row * Np);
        float v = 0.f;
        if (col < 8 * out_o) {
            const int j = (int)(row / in_o), m = (int)(row - (int64_t)j * in_o);
            const int i = col / out_o, n = col - i * out_o;
            const int w = i ^ j;
            const uint32_t byte = packed[((int64_t)w * out_o + n) * kp4 + m / 4];
            const int code = (int)((byte >> (6 - 2 * (m & 3))) & 3u) - 1;
            v = (float)(kOctSign[i][j] * code) * beta[n];
        }
        Act<T>::store(Bt + e, v);
    }
}

// dW and dbeta from C.  Threads [0, 8*out_o*in_o) take one dW element each;
// workgroups past that take one dbeta[n] each (256 threads, fixed-order tree).
__global__ __launch_bounds__(256) void octonion_fold_kernel(const float *__restrict__ C, int64_t ldc, int Sc,
                                                            int64_t cstride, const uint8_t *__restrict__ packed,
                                                            int in_o, int out_o, const float *__restrict__ beta,
                                                            const float *__restrict__ latent, float *__restrict__ dw,
                                                            float *__restrict__ db, int dw_blocks) {
    const int kp4 = (int)ceil_div(in_o, 4);
    if ((int)blockIdx.x < dw_blocks) {
        const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (!dw || e >= 8LL * out_o * in_o) return;
        const int m = (int)(e % in_o);
        const int64_t wn = e / in_o;
        const int n = (int)(wn % out_o), w = (int)(wn / out_o);
        double acc = 0.0;
        for (int i = 0; i < 8; ++i) {
            const int j = i ^ w;
            const int64_t off = (int64_t)(i * out_o + n) * ldc + (int64_t)j * in_o + m;
            double c = 0.0;
            for (int s = 0; s < Sc; ++s) c += (double)C[s * cstride + off];
            acc += kOctSign[i][j] * c;
        }
        float v = (float)(acc * (double)beta[n]);
        if (latent) {
            const float lw = latent[e];
            v = (lw >= -1.5f && lw <= 1.5f) ? v : 0.f;
        }
        dw[e] = v;
        return;
    }
    if (!db) return;
    __shared__ double part[256];
    const int n = (int)blockIdx.x - dw_blocks;
    double acc = 0.0;
    for (int e = threadIdx.x; e < 64 * in_o; e += blockDim.x) {  // e = (i*8 + j)*in_o + m
        const int m = e % in_o, ij = e / in_o, i = ij >> 3, j = ij & 7;
        const uint32_t byte = packed[((int64_t)(i ^ j) * out_o + n) * kp4 + m / 4];
        const int code = (int)((byte >> (6 - 2 * (m & 3))) & 3u) - 1;
        if (!code) continue;
        const int64_t off = (int64_t)(i * out_o + n) * ldc + (int64_t)j * in_o + m;
        double c = 0.0;
        for (int s = 0; s < Sc; ++s) c += (double)C[s * cstride + off];
        acc += (double)(kOctSign[i][j] * code) * c;
    }
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) part[threadIdx.x] += part[threadIdx.x + st];
        __syncthreads();
    }
    if (threadIdx.x == 0) db[n] = (float)part[0];
}

}  // namespace walsh

using namespace walsh;

WALSH_EXPORT int walsh_octonion_prepare_t(const uint8_t *packed, int64_t in_o, int64_t out_o, const float *beta,
                                          void *Bt, int dtype, void *stream) {
    if (!packed || !beta || !Bt) return set_error(WALSH_EINVAL, "walsh_octonion_prepare_t: null pointer");
    if (in_o <= 0 || out_o <= 0 || in_o > 65536 || out_o > 65536)
        return set_error(WALSH_EINVAL, "walsh_octonion_prepare_t: bad shape");
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "walsh_octonion_prepare_t: dtype");
    const int Np = (int)(ceil_div(8 * out_o, 32) * 32);
    const int64_t total = 8 * in_o * (int64_t)Np;
    int64_t grid = ceil_div(total, 256);
    if (grid > 8192) grid = 8192;
    if (dtype == WALSH_BF16)
        launch(octonion_expand_t_kernel<uint16_t>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, packed,
               (int)in_o, (int)out_o, beta, Np, (uint16_t *)Bt);
    else
        launch(octonion_expand_t_kernel<float>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, packed,
               (int)in_o, (int)out_o, beta, Np, (float *)Bt);
    return check_hip(hipGetLastError(), "walsh_octonion_prepare_t launch");
}

WALSH_EXPORT int walsh_octonion_bwd_fold(const float *C, int64_t ldc, int64_t n_parts, int64_t part_stride,
                                         const uint8_t *packed, int64_t in_o, int64_t out_o, const float *beta,
                                         const float *latent, float *dweight, float *dbeta, void *stream) {
    if (!C || !packed || !beta) return set_error(WALSH_EINVAL, "walsh_octonion_bwd_fold: null pointer");
    if (in_o <= 0 || out_o <= 0 || in_o > 65536 || out_o > 65536 || ldc < 8 * in_o || n_parts < 1 ||
        (n_parts > 1 && part_stride < 8 * out_o * ldc))
        return set_error(WALSH_EINVAL, "walsh_octonion_bwd_fold: bad shape");
    const int64_t nw = 8 * out_o * in_o;
    const int dw_blocks = dweight ? (int)ceil_div(nw, 256) : 0;
    const int64_t grid = dw_blocks + (dbeta ? out_o : 0);
    if (grid == 0) return WALSH_OK;
    launch(octonion_fold_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, C, ldc, (int)n_parts,
           part_stride, packed, (int)in_o, (int)out_o, beta, latent, dweight, dbeta, dw_blocks);
    return check_hip(hipGetLastError(), "walsh_octonion_bwd_fold launch");
}

// ------------------------------------------------------------------ weight-gradient product
// C = gy^T x ([8*out_o][8*in_o], K = tokens) on the forward's GEMM kernels:
// both operands are first transposed into token-contiguous rows (one pass
// each through a 64 x 64 LDS tile; rows padded with zeros to a multiple of
// 8 tokens), then a split-K GEMM writes float32
// partial sums, one slab per K split, which the fold adds in split order.
template <typename T>
__global__ __launch_bounds__(256) void octonion_transpose_kernel(const T *__restrict__ in, int64_t ldi, int R, int C,
                                                                 T *__restrict__ out, int64_t ldo) {
    // 4-element pieces both ways; odd row stride in 4-byte words keeps the
    // column reads on different banks
    __shared__ T tile[64][64 + (sizeof(T) == 2 ? 2 : 1)];
    const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
    const int tq = threadIdx.x & 15, tr = threadIdx.x >> 4;  // 16 pieces of 4 x 16 rows
#pragma unroll
    for (int r = tr; r < 64; r += 16) {
        const int rr = r0 + r, cc = c0 + 4 * tq;
        T v[4];
        if (rr < R && cc + 3 < C && (ldi & 3) == 0 && ((uintptr_t)in & (4 * sizeof(T) - 1)) == 0) {
            if constexpr (sizeof(T) == 2) {
                const uint2 u = *(const uint2 *)(in + (int64_t)rr * ldi + cc);
                v[0] = (T)(u.x & 0xffff); v[1] = (T)(u.x >> 16); v[2] = (T)(u.y & 0xffff); v[3] = (T)(u.y >> 16);
            } else {
                const f32x4 u = *(const f32x4 *)(in + (int64_t)rr * ldi + cc);
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = u[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = (rr < R && cc + j < C) ? in[(int64_t)rr * ldi + cc + j] : T(0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) tile[r][4 * tq + j] = v[j];
    }
    __syncthreads();
    // output row c (= input column), 4 consecutive input rows per thread;
    // columns R .. ldo-1 (the row padding) are written as zeros
#pragma unroll
    for (int c = tr; c < 64; c += 16) {
        const int cc = c0 + c, rr = r0 + 4 * tq;
        if (cc >= C || rr >= ldo) continue;
        T v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = tile[4 * tq + j][c];
        T *dst = out + (int64_t)cc * ldo + rr;
        if (rr + 3 < ldo) {
            if constexpr (sizeof(T) == 2)
                *(uint2 *)dst = uint2{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16)};
            else
                *(f32x4 *)dst = f32x4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (rr + j < ldo) dst[j] = v[j];
        }
    }
}

// C = the split-K partial sums added in split order (float32).
__global__ __launch_bounds__(256) void octonion_sum_parts_kernel(const float *__restrict__ parts, int S,
                                                                 int64_t stride, int64_t n, float *__restrict__ C) {
    for (int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; e < n;
         e += (int64_t)gridDim.x * blockDim.x * 4) {
        f32x4 acc = *(const f32x4 *)(parts + e);
        for (int sp = 1; sp < S; ++sp) acc += *(const f32x4 *)(parts + sp * stride + e);
        *(f32x4 *)(C + e) = acc;
    }
}

// split-K plan: about two work items per CU, splits of whole K stages and at
// least 4 stages each
static void octonion_dw_plan(int64_t M, int64_t in_o, int64_t out_o, bool bf16, int64_t *S, int64_t *kspan,
                             int64_t *Mp) {
    const int64_t N8o = 8 * out_o, N8i = 8 * in_o;
    const int64_t tiles = bf16 ? ceil_div(N8o, kOBM) * ceil_div(N8i, kOBN) : ceil_div(N8o, kBM) * ceil_div(N8i, kBN);
    const int64_t stage = bf16 ? kOBK : GemmCfg<float>::BK;
    int64_t s = ceil_div(2 * (int64_t)device_info().cu_count, tiles);
    const int64_t smax = ceil_div(M, 4 * stage);
    if (s > smax) s = smax;
    if (s < 1) s = 1;
    *kspan = ceil_div(ceil_div(M, s), stage) * stage;
    *S = ceil_div(M, *kspan);
    *Mp = ceil_div(M, 8) * 8;
}

static int64_t octonion_dw_ws(int64_t M, int64_t in_o, int64_t out_o, int dtype, int64_t *S, int64_t *kspan,
                              int64_t *Mp, int64_t *off_x, int64_t *off_c) {
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4;
    octonion_dw_plan(M, in_o, out_o, dtype == WALSH_BF16, S, kspan, Mp);
    *off_x = ceil_div(8 * out_o * *Mp * esz, 256) * 256;
    *off_c = *off_x + ceil_div(8 * in_o * *Mp * esz, 256) * 256;
    // partial sums [S][8 out_o][8 in_o], then (S > 1) their total
    return *off_c + (*S + (*S > 1 ? 1 : 0)) * 64 * out_o * in_o * 4;
}

WALSH_EXPORT int64_t walsh_octonion_bwd_params_workspace_bytes(int64_t M, int64_t in_o, int64_t out_o, int dtype) {
    if (M <= 0 || in_o <= 0 || out_o <= 0 || (dtype != WALSH_F32 && dtype != WALSH_BF16)) return 0;
    int64_t S, kspan, Mp, ox, oc;
    return octonion_dw_ws(M, in_o, out_o, dtype, &S, &kspan, &Mp, &ox, &oc);
}

WALSH_EXPORT int walsh_octonion_bwd_params(const void *gy, int64_t ldg, const void *x, int64_t ldx, int64_t M,
                                           int64_t in_o, int64_t out_o, const uint8_t *packed, const float *beta,
                                           const float *latent, float *dweight, float *dbeta, int dtype, void *work,
                                           int64_t work_bytes, void *stream) {
    const char *fn = "walsh_octonion_bwd_params";
    if (!gy || !x || !packed || !beta || !work) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M <= 0 || in_o <= 0 || out_o <= 0 || in_o > 65536 || out_o > 65536 || ldg < 8 * out_o || ldx < 8 * in_o)
        return set_error(WALSH_EINVAL, "%s: bad shape M=%lld in_o=%lld out_o=%lld", fn, (long long)M,
                         (long long)in_o, (long long)out_o);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype", fn);
    if (!dweight && !dbeta) return WALSH_OK;
    const bool bf16 = dtype == WALSH_BF16;
    const int64_t esz = bf16 ? 2 : 4;
    int64_t S, kspan, Mp, ox, oc;
    const int64_t need = octonion_dw_ws(M, in_o, out_o, dtype, &S, &kspan, &Mp, &ox, &oc);
    if (work_bytes < need || (uintptr_t)work % 256)
        return set_error(WALSH_EINVAL, "%s: workspace of %lld bytes (256-aligned), needs %lld", fn,
                         (long long)work_bytes, (long long)need);
    if (8 * out_o * Mp * esz > (int64_t)kMaxBufferBytes || 8 * in_o * Mp * esz > (int64_t)kMaxBufferBytes ||
        S * 64 * out_o * in_o * 4 > (int64_t)kMaxBufferBytes || M * ldg * esz > (int64_t)kMaxBufferBytes)
        return set_error(WALSH_ENOTSUP, "%s: operands above 2^31 bytes", fn);
    hipStream_t s = (hipStream_t)stream;
    char *w = (char *)work;
    void *gyT = w, *xT = w + ox;
    float *Cp = (float *)(w + oc);
    const dim3 tb(256);
    const dim3 tg_g((unsigned)ceil_div(8 * out_o, 64), (unsigned)ceil_div(M, 64));
    const dim3 tg_x((unsigned)ceil_div(8 * in_o, 64), (unsigned)ceil_div(M, 64));
    if (bf16) {
        launch(octonion_transpose_kernel<uint16_t>, tg_g, tb, 0, s, (const uint16_t *)gy, ldg, (int)M,
               (int)(8 * out_o), (uint16_t *)gyT, Mp);
        launch(octonion_transpose_kernel<uint16_t>, tg_x, tb, 0, s, (const uint16_t *)x, ldx, (int)M,
               (int)(8 * in_o), (uint16_t *)xT, Mp);
    } else {
        launch(octonion_transpose_kernel<float>, tg_g, tb, 0, s, (const float *)gy, ldg, (int)M, (int)(8 * out_o),
               (float *)gyT, Mp);
        launch(octonion_transpose_kernel<float>, tg_x, tb, 0, s, (const float *)x, ldx, (int)M, (int)(8 * in_o),
               (float *)xT, Mp);
    }
    OctArgs a{};
    a.x = gyT;
    a.ldx = Mp;
    a.M = (int)(8 * out_o);
    a.N = (int)(8 * in_o);
    a.K = (int)M;
    a.Kp = (int)Mp;
    a.B = xT;
    a.beta = nullptr;
    a.out_o = (int)(8 * in_o);
    a.y = Cp;
    a.ldy = 8 * in_o;
    a.splits = (int)S;
    a.kspan = kspan;
    a.ysplit = 64 * out_o * in_o;
    if (bf16) {
        gemm256_launch<kEpiF32>(a, s);
    } else {
        const dim3 G((unsigned)ceil_div(8 * out_o, kBM), (unsigned)ceil_div(8 * in_o, kBN), (unsigned)S);
        launch(octonion_gemm_kernel<float>, G, dim3(kGemmThreads), 0, s, a);
    }
    int rc = check_hip(hipGetLastError(), fn);
    if (rc) return rc;
    const int64_t nC = 64 * out_o * in_o;
    float *Ct = Cp;
    if (S > 1) {
        // one pass adds the partial sums, so the fold reads a single C
        Ct = Cp + S * nC;
        int64_t grid = ceil_div(nC / 4, 256);
        if (grid > 4096) grid = 4096;
        launch(octonion_sum_parts_kernel, dim3((unsigned)grid), dim3(256), 0, s, (const float *)Cp, (int)S, nC, nC, Ct);
        rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
    }
    return walsh_octonion_bwd_fold(Ct, 8 * in_o, 1, 0, packed, in_o, out_o, beta, latent, dweight, dbeta, stream);
}

WALSH_EXPORT int64_t walsh_octonion_weight_elems(int64_t in_o, int64_t out_o) {
    if (in_o <= 0 || out_o <= 0) return 0;
    return 8 * out_o * ceil_div(8 * in_o, 32) * 32;
}

WALSH_EXPORT int walsh_octonion_prepare(const uint8_t *packed, int64_t in_o, int64_t out_o, void *B, int dtype,
                                        void *stream) {
    if (!packed || !B) return set_error(WALSH_EINVAL, "walsh_octonion_prepare: null pointer");
    if (in_o <= 0 || out_o <= 0 || in_o > 65536 || out_o > 65536)
        return set_error(WALSH_EINVAL, "walsh_octonion_prepare: bad shape");
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "walsh_octonion_prepare: dtype");
    const int Kp = (int)(ceil_div(8 * in_o, 32) * 32);
    const int64_t total = 8 * out_o * (int64_t)Kp;
    const int block = 256;
    int64_t grid = ceil_div(total, block);
    if (grid > 8192) grid = 8192;
    if (dtype == WALSH_BF16)
        launch(octonion_expand_kernel<uint16_t>, dim3((unsigned)grid), dim3(block), 0, (hipStream_t)stream,
                           packed, (int)in_o, (int)out_o, Kp, (uint16_t *)B);
    else
        launch(octonion_expand_kernel<float>, dim3((unsigned)grid), dim3(block), 0, (hipStream_t)stream,
                           packed, (int)in_o, (int)out_o, Kp, (float *)B);
    return check_hip(hipGetLastError(), "walsh_octonion_prepare launch");
}

WALSH_EXPORT int walsh_octonion_linear_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                                           const void *B, const float *beta, void *y, int64_t ldy, int dtype,
                                           void *stream) {
    if (!x || !B || !y) return set_error(WALSH_EINVAL, "walsh_octonion_linear_fwd: null pointer");
    if (M < 0 || in_o <= 0 || out_o <= 0 || ldx < 8 * in_o || ldy < 8 * out_o)
        return set_error(WALSH_EINVAL, "walsh_octonion_linear_fwd: bad shape M=%lld in_o=%lld out_o=%lld",
                         (long long)M, (long long)in_o, (long long)out_o);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "walsh_octonion_linear_fwd: dtype");
    if (M == 0) return WALSH_OK;
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4;
    const int64_t vec = 16 / esz;
    if (ldx % vec || (uintptr_t)x % 16 || (uintptr_t)B % 16 || (8 * in_o) % vec)
        return set_error(WALSH_ENOTSUP, "walsh_octonion_linear_fwd: x/B must be 16-byte aligned rows");
    const int64_t N = 8 * out_o, K = 8 * in_o, Kp = ceil_div(K, 32) * 32;
    if (N * Kp * esz > (int64_t)kMaxBufferBytes) return set_error(WALSH_ENOTSUP, "walsh_octonion_linear_fwd: too large");
    const int64_t ld = ldx > ldy ? ldx : ldy;
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * esz) / kOBM * kOBM;
    if (rows_max < kOBM) return set_error(WALSH_ENOTSUP, "walsh_octonion_linear_fwd: row stride too large");
    rows_max = balanced_rows(M, rows_max, kOBM);
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        OctArgs a{};
        a.x = (const char *)x + r0 * ldx * esz;
        a.ldx = ldx;
        a.M = (int)rows;
        a.N = (int)N;
        a.K = (int)K;
        a.Kp = (int)Kp;
        a.B = B;
        a.beta = beta;
        a.out_o = (int)out_o;
        a.y = (char *)y + r0 * ldy * esz;
        a.ldy = ldy;
        if (dtype == WALSH_BF16) {
            gemm256_launch<kEpiBeta>(a, (hipStream_t)stream);
        } else {
            const dim3 G((unsigned)ceil_div(rows, kBM), (unsigned)ceil_div(N, kBN)), Bk(kGemmThreads);
            launch(octonion_gemm_kernel<float>, G, Bk, 0, (hipStream_t)stream, a);
        }
        const int rc = check_hip(hipGetLastError(), "walsh_octonion_linear_fwd launch");
        if (rc) return rc;
    }
    return WALSH_OK;
}

// The reference module's forward (OctonionFusedLinear.forward and
// OctonionPackedLinear.forward, cayley_dickson_cuda.py:650-668, :761-765): the
// fused kernel multiplies bf16 operands with float32 accumulation and returns
// bf16 (:402, :411, :421), and the module multiplies that by the float32 beta,
// which promotes to float32.  Here the rounding to bf16 and the beta product
// are the GEMM's epilogue, so y [M, ldy] float32 = float(bf16(x B^T)) * beta.
WALSH_EXPORT int walsh_octonion_fused_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                                          const void *B, const float *beta, float *y, int64_t ldy, void *stream) {
    const char *fn = "walsh_octonion_fused_fwd";
    if (!x || !B || !y) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || in_o <= 0 || out_o <= 0 || ldx < 8 * in_o || ldy < 8 * out_o)
        return set_error(WALSH_EINVAL, "%s: bad shape M=%lld in_o=%lld out_o=%lld", fn, (long long)M,
                         (long long)in_o, (long long)out_o);
    if (M == 0) return WALSH_OK;
    if (ldx % 8 || (8 * in_o) % 8 || (uintptr_t)x % 16 || (uintptr_t)B % 16 || ldy % 4 || (uintptr_t)y % 16)
        return set_error(WALSH_ENOTSUP, "%s: x/B/y must be 16-byte aligned rows", fn);
    const int64_t N = 8 * out_o, K = 8 * in_o, Kp = ceil_div(K, 32) * 32;
    if (N * Kp * 2 > (int64_t)kMaxBufferBytes) return set_error(WALSH_ENOTSUP, "%s: too large", fn);
    const int64_t row_bytes = ldx * 2 > ldy * 4 ? ldx * 2 : ldy * 4;
    int64_t rows_max = (int64_t)kMaxBufferBytes / row_bytes / kOBM * kOBM;
    if (rows_max < kOBM) return set_error(WALSH_ENOTSUP, "%s: row stride too large", fn);
    rows_max = balanced_rows(M, rows_max, kOBM);
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        OctArgs a{};
        a.x = (const char *)x + r0 * ldx * 2;
        a.ldx = ldx;
        a.M = (int)rows;
        a.N = (int)N;
        a.K = (int)K;
        a.Kp = (int)Kp;
        a.B = B;
        a.beta = beta;
        a.out_o = (int)out_o;
        a.y = y + r0 * ldy;
        a.ldy = ldy;
        gemm256_launch<kEpiBetaF32>(a, (hipStream_t)stream);
        const int rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
    }
    return WALSH_OK;
}
