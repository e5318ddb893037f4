// bf16 GEMM y[m][n] = epi(sum_k x[m][k] B[n][k]) on 256 x 256 output tiles
// (the octonion forward and the wide MoE router's first layer).
#pragma once
#include "common.h"

namespace walsh {

struct Gemm256Args {
    const void *x;
    int64_t ldx;
    int M, N, K, Kp;     // K = columns of x used, Kp = B row length (>= K)
    const void *B;       // [N][Kp]
    const float *beta;   // kEpiBeta: column n scaled by beta[n % out_o] (null: 1)
    int out_o;
    void *y;
    int64_t ldy;
    // split-K (kspan > 0): split s sums columns [s kspan, (s+1) kspan) and
    // writes its own output ysplit elements after split s-1's
    int splits;
    int64_t kspan, ysplit;
};

// epilogues: beta scaling to bf16 (octonion forward), SiLU of the bf16-rounded
// product to bf16 (router), plain float32 (split-K partial sums)
enum { kEpiBeta = 0, kEpiSilu = 1, kEpiF32 = 2 };

// Round to the nearest bfloat16 and back: where the reference runs under
// bf16 autocast, every Linear/einsum output and elementwise result is a
// bf16 tensor, so the bf16 paths round at the same points.
__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }
__device__ __forceinline__ float silu_f(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// ------------------------------------------------------- bf16 GEMM, 256 x 256
// The bf16 forward at every shape.  256 x 256 output tiles, 8 wavefronts of
// 64 outputs x 128 tokens each.  The product runs transposed, D[n][m] =
// sum_k B[n][k] x[m][k] on 16x16x32 bf16 MFMA, so a lane's accumulator holds
// 4 consecutive outputs of one token: the epilogue writes 8-byte pieces of
// rows with beta applied.
//   * Per 64-wide K stage both operand tiles (x: 256 tokens, the dense +-1/0
//     block matrix: 256 outputs; 32 KB each) go global -> registers -> LDS,
//     double buffered with one barrier per stage; every global byte is
//     fetched once per workgroup (two wavefronts share each weight row, four
//     each x row).
//   * LDS rows are 128 B with the 16-byte chunks XOR-swizzled by the row
//     (chunk ^ (row & 7)), so fragment reads and tile stores are free of bank
//     conflicts (measured with SQ_LDS_BANK_CONFLICT).
//   * Tiles are numbered XCD-major: workgroup b runs on XCD b % 8, and takes
//     tile (b % 8) * per_xcd + b / 8, so the output tiles of one row block run
//     side by side on one XCD and x comes from HBM once into that XCD's L2.
constexpr int kOBM = 256, kOBN = 256, kOBK = 64;
constexpr int kOThreads = 512;
constexpr int kOTile = kOBM * 128;  // bytes of one staged operand tile

// byte offset of 16-byte chunk `part` (0..7) of staged row `row`
__device__ __forceinline__ int oct_off(int row, int part) { return row * 128 + ((part ^ (row & 7)) << 4); }

template <int EPI>
__device__ __forceinline__ void gemm256_body(const Gemm256Args &a, int nM, int nN, int per_xcd) {
    __shared__ __align__(16) unsigned char lds[2][2][kOTile];  // [buffer][x | weights]

    int tile = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
    const int splits = a.splits > 0 ? a.splits : 1;
    if (tile >= nM * nN * splits) return;
    const int split = tile / (nM * nN);
    tile -= split * nM * nN;
    const int k_lo = a.kspan > 0 ? (int)(split * a.kspan) : 0;
    const int k_hi = a.kspan > 0 ? (int)(k_lo + a.kspan < a.K ? k_lo + a.kspan : a.K) : a.K;
    const int mb = tile / nN, nb = tile - mb * nN;
    const int m0 = mb * kOBM, n0 = nb * kOBN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wn = wave & 3, wm = wave >> 2;
    const int fr = lane & 15, fq = lane >> 4;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * 2));
    const __amdgpu_buffer_rsrc_t br = make_rsrc(a.B, (uint32_t)((int64_t)a.N * a.Kp * 2));

    // staging: each operand tile is 256 rows x 8 chunks of 16 B; thread takes
    // chunk tid + 512 i (i = 0..3) of both: row (tid >> 3) + 64 i, chunk
    // tid & 7.  Out-of-range chunks read zeros.
    const int srow = tid >> 3, spart = tid & 7;
    auto load = [&](int k0, u32x4 (&xst)[4], u32x4 (&wst)[4]) {
        const int k = k_lo + k0 + spart * 8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + srow + 64 * i, n = n0 + srow + 64 * i;
            xst[i] = __builtin_amdgcn_raw_buffer_load_b128(
                xr, (m < a.M && k < k_hi) ? (uint32_t)(((int64_t)m * a.ldx + k) * 2) : kOOB, 0, 0);
            wst[i] = __builtin_amdgcn_raw_buffer_load_b128(
                br, (n < a.N && k < (a.kspan > 0 ? k_hi : a.Kp)) ? (uint32_t)(((int64_t)n * a.Kp + k) * 2) : kOOB,
                0, 0);
        }
    };
    auto store = [&](int buf, const u32x4 (&xst)[4], const u32x4 (&wst)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int off = oct_off(srow + 64 * i, spart);
            *(u32x4 *)(&lds[buf][0][off]) = xst[i];
            *(u32x4 *)(&lds[buf][1][off]) = wst[i];
        }
    };

    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Stage st + 2 is fetched during stage st into the register set stage
    // st + 1 was stored from, so each global load has two stages of products
    // to land in; sched_barrier(0) keeps the compiler from sinking the
    // prefetch below the products.
    auto stage = [&](int st, u32x4 (&xn)[4], u32x4 (&wn_)[4], u32x4 (&xf_)[4], u32x4 (&wf_)[4]) {
        const int cur = st & 1;
        load((st + 2) * kOBK, xf_, wf_);  // zeros past the end
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            u32x4 wf[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) wf[t] = *(const u32x4 *)(&lds[cur][1][oct_off(wn * 64 + t * 16 + fr, sub * 4 + fq)]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // the wave's 8 token tiles in two halves (register pressure)
                u32x4 xf[4];
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    xf[t] = *(const u32x4 *)(&lds[cur][0][oct_off(wm * 128 + (h * 4 + t) * 16 + fr, sub * 4 + fq)]);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[i][h * 4 + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, wf[i]), __builtin_bit_cast(bf16x8, xf[j]), acc[i][h * 4 + j], 0,
                            0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        store(cur ^ 1, xn, wn_);            // stage st + 1
        __syncthreads();
    };

    const int nst = (int)ceil_div(k_hi - k_lo, kOBK);
    u32x4 xa[4], wa[4], xb[4], wb[4];
    load(0, xa, wa);
    load(kOBK, xb, wb);
    store(0, xa, wa);
    __syncthreads();
    int st = 0;
    for (; st + 1 < nst; st += 2) {
        stage(st, xb, wb, xa, wa);
        stage(st + 1, xa, wa, xb, wb);
    }
    if (st < nst) stage(st, xb, wb, xa, wa);

    // epilogue: acc[i][j][r] = D[n = 16 i + 4 fq + r][m = 16 j + fr] of the wave's tile
    if constexpr (EPI == kEpiF32) {
        const int64_t span = a.kspan > 0 ? (int64_t)(splits - 1) * a.ysplit + (int64_t)a.M * a.ldy : (int64_t)a.M * a.ldy;
        const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)(span * 4));
        const int64_t ybase = (int64_t)split * a.ysplit;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + wn * 64 + i * 16 + fq * 4;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int m = m0 + wm * 128 + j * 16 + fr;
                const uint32_t off = (m < a.M && n < a.N) ? (uint32_t)((ybase + (int64_t)m * a.ldy + n) * 4) : kOOB;
                Buf4<float>::store(acc[i][j], yr, off, 0);
            }
        }
        return;
    }
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * 2));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = n0 + wn * 64 + i * 16 + fq * 4;
        f32x4 bv = f32x4{0.f, 0.f, 0.f, 0.f};
        if (EPI == kEpiBeta && n < a.N) {
#pragma unroll
            for (int r = 0; r < 4; ++r) bv[r] = a.beta ? a.beta[(n + r) % a.out_o] : 1.f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int m = m0 + wm * 128 + j * 16 + fr;
            const uint32_t off = (m < a.M && n < a.N) ? (uint32_t)(((int64_t)m * a.ldy + n) * 2) : kOOB;
            if constexpr (EPI == kEpiBeta) {
                Buf4<uint16_t>::store(acc[i][j] * bv, yr, off, 0);
            } else {
                // the product rounded to bf16, SiLU on that value, rounded again
                f32x4 v;
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = silu_f(bf16r(acc[i][j][r]));
                Buf4<uint16_t>::store(v, yr, off, 0);
            }
        }
    }
}

static __global__ __launch_bounds__(kOThreads, 1) void gemm256_beta_kernel(Gemm256Args a, int nM, int nN, int per_xcd) {
    gemm256_body<kEpiBeta>(a, nM, nN, per_xcd);
}
static __global__ __launch_bounds__(kOThreads, 1) void gemm256_silu_kernel(Gemm256Args a, int nM, int nN, int per_xcd) {
    gemm256_body<kEpiSilu>(a, nM, nN, per_xcd);
}
static __global__ __launch_bounds__(kOThreads, 1) void gemm256_f32_kernel(Gemm256Args a, int nM, int nN, int per_xcd) {
    gemm256_body<kEpiF32>(a, nM, nN, per_xcd);
}

// grid: ceil(M / 256) x ceil(N / 256) tiles (x splits) in XCD-major order
template <int EPI>
static inline void gemm256_launch(const Gemm256Args &a, hipStream_t s) {
    const int nM = (int)ceil_div(a.M, kOBM), nN = (int)ceil_div(a.N, kOBN);
    const int per_xcd = (int)ceil_div((int64_t)nM * nN * (a.splits > 0 ? a.splits : 1), 8);
    if constexpr (EPI == kEpiBeta)
        launch(gemm256_beta_kernel, dim3((unsigned)(per_xcd * 8)), dim3(kOThreads), 0, s, a, nM, nN, per_xcd);
    else if constexpr (EPI == kEpiSilu)
        launch(gemm256_silu_kernel, dim3((unsigned)(per_xcd * 8)), dim3(kOThreads), 0, s, a, nM, nN, per_xcd);
    else
        launch(gemm256_f32_kernel, dim3((unsigned)(per_xcd * 8)), dim3(kOThreads), 0, s, a, nM, nN, per_xcd);
}

}  // namespace walsh
