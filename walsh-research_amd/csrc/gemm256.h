// bf16 GEMM y[m][n] = epi(sum_k x[m][k] B[n][k]) on 256 x 256 output tiles
// (the octonion forward and weight gradient, the wide MoE router's first layer).
#pragma once
#include <type_traits>

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
// product to bf16 (router), plain float32 (split-K partial sums), the product
// rounded to bf16 and then scaled by beta in float32, stored as float32 (the
// octonion module's output: a bf16 kernel result times a float32 parameter)
enum { kEpiBeta = 0, kEpiSilu = 1, kEpiF32 = 2, kEpiBetaF32 = 3 };

// Round to the nearest bfloat16 and back: where the reference runs under
// bf16 autocast, every Linear/einsum output and elementwise result is a
// bf16 tensor, so the bf16 paths round at the same points.
__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }
__device__ __forceinline__ float silu_f(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// ------------------------------------------------------- bf16 GEMM, 256 x 256
// Persistent workgroups of 4 wavefronts (one per SIMD), each wavefront 128
// outputs x 128 tokens, so a K step of 32 costs 16 fragment reads from LDS
// per 64 MFMA (16x16x32 bf16).  The product runs transposed, D[n][m] =
// sum_k B[n][k] x[m][k], so a lane's accumulator holds 4 consecutive outputs
// of one token and the epilogue writes 8- or 16-byte pieces of rows.  The
// 64 accumulator tiles (256 registers a lane) live in the AGPR half of the
// register file.
//   * Operands move global -> LDS with buffer_load_dwordx4 ... lds (no VGPR
//     round trip).  A super-stage is 64 columns of both 256-row tiles, 128
//     bytes a row (whole cache lines: half-line requests halved the L2
//     throughput), 64 KB; two of them fit the LDS.  Each load instruction
//     fills 1 KB = 8 rows; lane l lands at byte 16 l of it, so lane l
//     fetches row l >> 3, chunk (l & 7) ^ (row & 7): 16-byte chunk c of row
//     r sits at position c ^ (r & 7), and fragment reads (8 lanes per LDS
//     cycle, rows r..r+7 of one chunk) are free of bank conflicts.
//   * K runs in sub-stages of 32 columns (half a super-stage): the
//     fragments of sub-stage t + 1 are read (interleaved with the products,
//     two reads per eight MFMA) while the products of t run from registers.
//     At every odd sub-stage 2S + 1 the workgroup waits for super-stage S + 1
//     and synchronises once; super-stage S's buffer is then free (its last
//     fragments are in registers) and super-stage S + 2 is issued into it,
//     interleaved with that sub-stage's products, two sub-stages ahead of use.
//   * The load stream runs across work items, so the next item's first
//     super-stages are in flight while an item's epilogue stores.
//   * Work items (tile, split) are numbered XCD-major: item w runs on XCD
//     w / per_xcd (workgroup b lives on XCD b % 8), so the output tiles of one
//     row block run side by side on one XCD and x comes from HBM about once
//     into that XCD's L2.
constexpr int kOBM = 256, kOBN = 256, kOBK = 64;  // tile rows of x, rows of B, columns per super-stage
constexpr int kOThreads = 256;
constexpr int kORow = 128;         // bytes of one staged row
constexpr int kOOp = 256 * kORow;  // one operand of a super-stage
constexpr int kOStage = 2 * kOOp;  // both operands: 64 KB

struct Gemm256Plan {
    int nM, nN, items, per_xcd, wg_per_xcd, nss;  // nss: super-stages per item
};

// position of 16-byte chunk c of staged row r
__device__ __forceinline__ int g256_pos(int r, int c) { return c ^ (r & 7); }

template <int EPI>
__device__ __forceinline__ void gemm256_body(const Gemm256Args &a, const Gemm256Plan &p) {
    __shared__ __align__(1024) unsigned char lds[2 * kOStage];

    const int xcd = (int)(blockIdx.x % 8), wgi = (int)(blockIdx.x / 8);
    const int first = xcd * p.per_xcd + wgi;
    const int end = min((xcd + 1) * p.per_xcd, p.items);
    if (first >= end) return;
    const int n_items = (end - first + p.wg_per_xcd - 1) / p.wg_per_xcd;  // items first, first + wg_per_xcd, ..
    const int tiles = p.nM * p.nN;

    const int tid = threadIdx.x, lane = tid & 63, fr = lane & 15, fq = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;

    // work item r of this workgroup: output tile and K range
    struct Item {
        int m0, n0, k_lo, k_hi, split;
    };
    auto item = [&](int r) {
        Item it;
        const int w = first + r * p.wg_per_xcd;
        it.split = w / tiles;
        const int tile = w - it.split * tiles;
        const int mb = tile / p.nN;
        it.m0 = mb * kOBM;
        it.n0 = (tile - mb * p.nN) * kOBN;
        if (a.kspan > 0) {
            it.k_lo = (int)(it.split * a.kspan);
            it.k_hi = (int)min((int64_t)a.K, (int64_t)it.k_lo + a.kspan);
        } else {
            it.k_lo = 0;
            it.k_hi = a.K;
        }
        return it;
    };

    // loads: waves 0, 1 stage x rows 128 (wave & 1) .. +127 of the tile, waves
    // 2, 3 the B rows; instruction i (0..15) covers rows 8 i .. 8 i + 7 of them
    const bool xrole = wave < 2;
    const __amdgpu_buffer_rsrc_t rs = xrole ? make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * 2))
                                            : make_rsrc(a.B, (uint32_t)((int64_t)a.N * a.Kp * 2));
    const uint32_t ld2 = (uint32_t)((xrole ? a.ldx : (int64_t)a.Kp) * 2);
    const int lim = xrole ? a.M : a.N;
    const int dch = (lane & 7) ^ (lane >> 3);
    const int lrow = (wave & 1) * 128 + (lane >> 3);
    const int opoff = (xrole ? 0 : kOOp) + (wave & 1) * 16 * 1024;
    // super-stage G of the workgroup's stream (item G / nss): per-lane byte
    // offset of instruction 0 (kOOB when nothing is to load) and whether
    // instruction i's row exists (row + 8 i < lim)
    struct Src {
        uint32_t off;
        int rows_left;
    };
    auto src = [&](int G) {
        Src s;
        const int r = G / p.nss, S = G - r * p.nss;
        s.off = kOOB;
        s.rows_left = 0;
        if (r < n_items) {
            const Item it = item(r);
            const int row = (xrole ? it.m0 : it.n0) + lrow;
            const int k = it.k_lo + S * kOBK + dch * 8;
            if (k < it.k_hi && row < lim) {
                s.off = (uint32_t)row * ld2 + (uint32_t)k * 2;
                s.rows_left = lim - row;
            }
        }
        return s;
    };
    auto dma = [&](int G, const Src &s, int i) {
        unsigned char *dst = lds + (G & 1) * kOStage + opoff + i * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16,
                                                 8 * i < s.rows_left ? s.off + (uint32_t)(8 * i) * ld2 : kOOB, 0, 0,
                                                 0);
    };
    // fragments of sub-stage t: super-stage t / 2, chunks 4 (t & 1) + fq
    auto rd = [&](int t, int g, u32x4 &bf, u32x4 &xf) {
        const unsigned char *base = lds + ((t >> 1) & 1) * kOStage;
        const int c = 4 * (t & 1) + fq;
        const int rb = wn * 128 + g * 16 + fr, rx = wm * 128 + g * 16 + fr;
        bf = *(const u32x4 *)(base + kOOp + rb * kORow + (g256_pos(rb, c) << 4));
        xf = *(const u32x4 *)(base + rx * kORow + (g256_pos(rx, c) << 4));
    };

    f32x4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // epilogue of item r: acc[i][j][q] = D[n = n0 + 128 wn + 16 i + 4 fq + q][m = m0 + 128 wm + 16 j + fr]
    auto epilogue = [&](int r) {
        const Item it = item(r);
        if constexpr (EPI == kEpiBetaF32) {
            const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * 4));
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int n = it.n0 + wn * 128 + i * 16 + fq * 4;
                f32x4 bv = f32x4{1.f, 1.f, 1.f, 1.f};
                if (a.beta && n < a.N) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) bv[q] = a.beta[(n + q) % a.out_o];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int m = it.m0 + wm * 128 + j * 16 + fr;
                    const uint32_t off = (m < a.M && n < a.N) ? (uint32_t)(((int64_t)m * a.ldy + n) * 4) : kOOB;
                    f32x4 v;
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] = bf16r(acc[i][j][q]) * bv[q];
                    Buf4<float>::store(v, yr, off, 0);
                }
            }
        } else if constexpr (EPI == kEpiF32) {
            const int64_t span = a.kspan > 0 ? (int64_t)(p.items / tiles - 1) * a.ysplit + (int64_t)a.M * a.ldy
                                             : (int64_t)a.M * a.ldy;
            const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)(span * 4));
            const int64_t ybase = a.kspan > 0 ? (int64_t)it.split * a.ysplit : 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int n = it.n0 + wn * 128 + i * 16 + fq * 4;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int m = it.m0 + wm * 128 + j * 16 + fr;
                    const uint32_t off =
                        (m < a.M && n < a.N) ? (uint32_t)((ybase + (int64_t)m * a.ldy + n) * 4) : kOOB;
                    Buf4<float>::store(acc[i][j], yr, off, 0);
                }
            }
        } else {
            const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * 2));
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int n = it.n0 + wn * 128 + i * 16 + fq * 4;
                f32x4 bv = f32x4{1.f, 1.f, 1.f, 1.f};
                if (EPI == kEpiBeta && a.beta && n < a.N) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) bv[q] = a.beta[(n + q) % a.out_o];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int m = it.m0 + wm * 128 + j * 16 + fr;
                    const uint32_t off = (m < a.M && n < a.N) ? (uint32_t)(((int64_t)m * a.ldy + n) * 2) : kOOB;
                    if constexpr (EPI == kEpiBeta) {
                        Buf4<uint16_t>::store(acc[i][j] * bv, yr, off, 0);
                    } else {
                        // the product rounded to bf16, SiLU on that value, rounded again
                        f32x4 v;
#pragma unroll
                        for (int q = 0; q < 4; ++q) v[q] = silu_f(bf16r(acc[i][j][q]));
                        Buf4<uint16_t>::store(v, yr, off, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // prologue: super-stages 0 and 1 in flight, wait for 0
    {
        const Src s0 = src(0), s1 = src(1);
#pragma unroll
        for (int i = 0; i < 16; ++i) dma(0, s0, i);
#pragma unroll
        for (int i = 0; i < 16; ++i) dma(1, s1, i);
    }
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    u32x4 b0[8], x0[8], b1[8], x1[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) rd(0, g, b0[g], x0[g]);

    // sub-stage t (of the workgroup's stream; 2 nss per item): products of t
    // from registers while the fragments of t + 1 are read.  The previous
    // sub-stage's reads are complete (lgkmcnt(0); they were issued a whole
    // sub-stage ago).  Odd t: super-stage (t + 1) / 2 has landed (nothing was
    // issued after it but stores), and once every wave is past the barrier
    // none reads the buffer of super-stage (t - 1) / 2, which takes
    // super-stage (t - 1) / 2 + 2.
    auto step = [&](int t, const u32x4 (&bc)[8], const u32x4 (&xc)[8], u32x4 (&bn)[8], u32x4 (&xn)[8], auto odd) {
        constexpr bool ODD = decltype(odd)::value;
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        Src s{kOOB, 0};
        const int G = (t - 1) / 2 + 2;
        if constexpr (ODD) {
            s = src(G);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            asm volatile("s_barrier" ::: "memory");
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            if constexpr (ODD) {
                dma(G, s, 2 * g);
                dma(G, s, 2 * g + 1);
            }
            rd(t + 1, g, bn[g], xn[g]);  // past the stream's end: unused values
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, bc[g]),
                                                                    __builtin_bit_cast(bf16x8, xc[j]), acc[g][j], 0,
                                                                    0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    const int per_item = 2 * p.nss;
    for (int r = 0; r < n_items; ++r) {
        const int t0 = r * per_item;
        for (int t = t0; t < t0 + per_item; t += 2) {
            step(t, b0, x0, b1, x1, std::false_type{});
            step(t + 1, b1, x1, b0, x0, std::true_type{});
        }
        epilogue(r);
        // the next item's first fragments again (its super-stage landed before
        // the last barrier): the values read by the last step are not kept
        // across the epilogue
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
#pragma unroll
        for (int g = 0; g < 8; ++g) rd(t0 + per_item, g, b0[g], x0[g]);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS write may outlive the workgroup
}

static __global__ __launch_bounds__(kOThreads, 1) void gemm256_beta_kernel(Gemm256Args a, Gemm256Plan p) {
    gemm256_body<kEpiBeta>(a, p);
}
static __global__ __launch_bounds__(kOThreads, 1) void gemm256_silu_kernel(Gemm256Args a, Gemm256Plan p) {
    gemm256_body<kEpiSilu>(a, p);
}
static __global__ __launch_bounds__(kOThreads, 1) void gemm256_f32_kernel(Gemm256Args a, Gemm256Plan p) {
    gemm256_body<kEpiF32>(a, p);
}
static __global__ __launch_bounds__(kOThreads, 1) void gemm256_beta_f32_kernel(Gemm256Args a, Gemm256Plan p) {
    gemm256_body<kEpiBetaF32>(a, p);
}

// Requirements (checked by the callers): K % 8 == 0, N % 4 == 0, ldx and Kp
// multiples of 8, x / B / y within 2^31 bytes, 16-byte aligned operands.
static inline Gemm256Plan gemm256_plan(const Gemm256Args &a) {
    Gemm256Plan p;
    p.nM = (int)ceil_div(a.M, kOBM);
    p.nN = (int)ceil_div(a.N, kOBN);
    p.items = p.nM * p.nN * (a.splits > 0 ? a.splits : 1);
    p.nss = (int)ceil_div(a.kspan > 0 ? a.kspan : (int64_t)a.K, kOBK);
    p.per_xcd = (int)ceil_div(p.items, 8);
    const int per_xcd_cus = device_info().cu_count / 8 > 0 ? device_info().cu_count / 8 : 1;
    p.wg_per_xcd = p.per_xcd < per_xcd_cus ? p.per_xcd : per_xcd_cus;
    return p;
}

// one workgroup per CU at most (128 KB of LDS each), items XCD-major
template <int EPI>
static inline void gemm256_launch(const Gemm256Args &a, hipStream_t s) {
    const Gemm256Plan p = gemm256_plan(a);
    if (p.items == 0 || p.nss == 0) return;
    const dim3 grid((unsigned)(8 * p.wg_per_xcd)), block(kOThreads);
    if constexpr (EPI == kEpiBeta)
        launch(gemm256_beta_kernel, grid, block, 0, s, a, p);
    else if constexpr (EPI == kEpiSilu)
        launch(gemm256_silu_kernel, grid, block, 0, s, a, p);
    else if constexpr (EPI == kEpiBetaF32)
        launch(gemm256_beta_f32_kernel, grid, block, 0, s, a, p);
    else
        launch(gemm256_f32_kernel, grid, block, 0, s, a, p);
}

}  // namespace walsh
