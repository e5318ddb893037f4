// Device helpers shared by the Hadamard-32 forward and backward kernels:
// the 32-point transform over groups, the launch arguments, the lane
// layout loads/transforms of activation rows and the per-group ternary
// matrix-core contraction (layouts documented at each helper).
#pragma once

#include "common.h"

#include <type_traits>

namespace walsh {

constexpr int kTile = 16;       // tokens per wavefront tile
constexpr int kWaves = 4;       // wavefronts per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kKChunk = 16;     // input columns per chunk (4 per lane)
constexpr int kNTile = 16;      // output columns per matrix-core tile

// ---------------------------------------------------------------- helpers

// Unnormalised 32-point Walsh-Hadamard transform along the group index of
// independent columns held as v[g][j] (Sylvester ordering, in place).
template <typename V>
__device__ __forceinline__ void fht32(V (&v)[32]) {
#pragma unroll
    for (int h = 1; h < 32; h <<= 1) {
#pragma unroll
        for (int g = 0; g < 32; ++g) {
            if (g & h) continue;
            const V a = v[g];
            const V b = v[g + h];
            v[g] = a + b;
            v[g + h] = a - b;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

__device__ __forceinline__ void fht32x4(f32x4 (&v)[32]) { fht32<f32x4>(v); }

struct HadArgs {
    const void *x;      // first row of this launch
    int64_t ldx;
    int M;              // rows of this launch (M * ldx * esize < 2^31)
    int in_o, out_o, Nt, Kc;
    int gsx, gsy;       // group strides of x / y rows (>= in_o / out_o)
    const uint8_t *kw;
    const uint8_t *kw3;  // base-3 layout (wide bf16 kernel), or null
    const float *alpha;  // [32][in_o]; null: all ones
    const float *beta;   // row h of beta at beta + h * beta_h
    int beta_h;          // out_o, or 0 for one beta row shared by all groups
    void *y;
    int64_t ldy;
    // x rows in batches (0: plain rows at ldx): row r sits at
    // (r / tpb) * bstride + (r % tpb) * ldx elements; xspan is the element
    // extent of x those rows cover (the batch stride alone says nothing of
    // it: a size-1 batch dimension may carry any stride)
    int tpb;
    int64_t bstride;
    int64_t xspan;
    // rotary embedding on the outputs (null: none): pairs (2i, 2i+1) of each
    // rope_D-wide head turn by rope[t][i] = (cos, sin), t = row % rope_T
    const float *rope;
    int rope_T, rope_D;
    int rope_row0;  // row 0 of this launch is row rope_row0 of a sequence
    // waves of a workgroup that take tiles (1..4; 0 means all 4).  With
    // fewer tiles than wavefronts on the chip, one working wave per
    // workgroup spreads the tiles over every CU instead of a quarter of them.
    int wave_tiles;
    // non-temporal output stores (whole-row variant): outputs far larger
    // than the caches, which a later kernel would read from HBM anyway
    int nt_store;
};

// A kernel reads its arguments with scalar loads placed where each field is
// first used, and in a latency-bound launch (decode sizes) every such load
// that misses the caches waits a memory round trip of its own, in sequence
// with the branches between them.  Reading every field at entry and passing
// the values through an empty asm statement (which the compiler cannot
// re-read from argument memory) leaves a single round trip for all of them.
__device__ __forceinline__ HadArgs load_args(const HadArgs &src) {
    HadArgs a = src;
    asm volatile("" : "+s"(a.x), "+s"(a.ldx), "+s"(a.M), "+s"(a.in_o), "+s"(a.out_o), "+s"(a.Nt), "+s"(a.Kc),
                 "+s"(a.gsx), "+s"(a.gsy), "+s"(a.kw), "+s"(a.kw3), "+s"(a.alpha), "+s"(a.beta), "+s"(a.beta_h));
    asm volatile("" : "+s"(a.y), "+s"(a.ldy), "+s"(a.tpb), "+s"(a.bstride), "+s"(a.xspan), "+s"(a.rope),
                 "+s"(a.rope_T), "+s"(a.rope_D), "+s"(a.rope_row0), "+s"(a.wave_tiles), "+s"(a.nt_store));
    return a;
}

// The (cos, sin) of the lane's two output pairs o0..o0+3 (o0 % 4 == 0,
// rope_D % 4 == 0, out_o % rope_D == 0: the same pairs in every group).
__device__ __forceinline__ f32x4 rope_cs(const HadArgs &a, int row, int o0) {
    const int t = (row + a.rope_row0) % a.rope_T, i0 = (o0 % a.rope_D) >> 1;
    return *(const f32x4 *)(a.rope + ((int64_t)t * (a.rope_D >> 1) + i0) * 2);
}

// One pair (e, o) turned by (c, s) with the fused multiply-adds written out:
// e c - o s as fma(e, c, -(o s)) and e s + o c as fma(e, s, o c).  The
// kernels that rotate whole fragments (rope_apply) leave the contraction to
// the compiler, which forms exactly these two (checked in the gfx950 code and
// by the tests that compare the decode-sized kernel, which uses these, with
// the wide kernel bitwise); writing them out there instead made the wide
// kernel spill.
__device__ __forceinline__ float rope_even(float e, float o, float c, float s) { return __builtin_fmaf(e, c, -(o * s)); }
__device__ __forceinline__ float rope_odd(float e, float o, float c, float s) { return __builtin_fmaf(e, s, o * c); }

__device__ __forceinline__ f32x4 rope_apply(f32x4 r, f32x4 cs) {
    return f32x4{r[0] * cs[0] - r[1] * cs[1], r[0] * cs[1] + r[1] * cs[0], r[2] * cs[2] - r[3] * cs[3],
                 r[2] * cs[3] + r[3] * cs[2]};
}

__device__ __forceinline__ uint32_t x_row_off(const HadArgs &a, int row, uint32_t esz) {
    const int64_t e = a.tpb ? (int64_t)(row / a.tpb) * a.bstride + (int64_t)(row % a.tpb) * a.ldx : (int64_t)row * a.ldx;
    return (uint32_t)(e * esz);
}

__device__ __forceinline__ uint32_t x_bytes(const HadArgs &a, uint32_t esz) {
    const int64_t e = a.tpb ? a.xspan : (int64_t)a.M * a.ldx;
    return (uint32_t)(e * esz);
}

// Transformed inputs of the lane's 4 columns over the 32 groups.
template <bool BF16MMA> struct XM;
template <> struct XM<false> { f32x4 v[32]; };
template <> struct XM<true> { uint2 b[32]; };

// LDS layout (all 16-byte entries, lane-major so each lane walks its 32
// groups with immediate offsets):
//   lut     [256]            code byte -> 4 weights (bf16x4 in 8 B, or f32x4)
//   alpha_l [Kc][4][32]      alpha[g, 16c+4q .. +3]   (0 past in_o)
//   beta_l  [Nt][4][32]      beta[h, 16nt+4q .. +3]/32 (0 past out_o)
template <bool BF16MMA> constexpr int lut_bytes() { return BF16MMA ? 256 * 8 : 256 * 16; }

// The lane's 4 columns 16c+4q.. of all 32 groups of its row (zeros past
// in_o / M).
template <typename T, bool VEC>
__device__ __forceinline__ void load_x(const HadArgs &a, __amdgpu_buffer_rsrc_t xr, uint32_t row_off, bool row_ok,
                                       int c, int q, f32x4 (&v)[32]) {
    constexpr uint32_t esz = sizeof(T);
    const int i0 = kKChunk * c + 4 * q;
    const uint32_t gstride = (uint32_t)a.gsx * esz;
    if (VEC) {
        const uint32_t voff = (row_ok && i0 < a.in_o) ? row_off + (uint32_t)i0 * esz : kOOB;
#pragma unroll
        for (int g = 0; g < 32; ++g) v[g] = Buf4<T>::load(xr, voff, (uint32_t)g * gstride);
    } else {
        uint32_t voff[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) voff[j] = (row_ok && i0 + j < a.in_o) ? row_off + (uint32_t)(i0 + j) * esz : kOOB;
#pragma unroll
        for (int g = 0; g < 32; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) v[g][j] = Buf4<T>::load1(xr, voff[j], (uint32_t)g * gstride);
    }
}

template <typename T, bool BF16MMA, bool VEC>
__device__ __forceinline__ void load_transform(const HadArgs &a, __amdgpu_buffer_rsrc_t xr, uint32_t row_off,
                                               bool row_ok, int c, int q, const f32x4 *__restrict__ alpha_l,
                                               XM<BF16MMA> &out) {
    f32x4 v[32];
    load_x<T, VEC>(a, xr, row_off, row_ok, c, q, v);
    const f32x4 *al = alpha_l + (c * 4 + q) * 32;
#pragma unroll
    for (int g = 0; g < 32; ++g) {
        v[g] = v[g] * al[g];
        if ((g & 7) == 7) __builtin_amdgcn_sched_barrier(0);
    }
    fht32x4(v);
    if constexpr (BF16MMA) {
#pragma unroll
        for (int g = 0; g < 32; ++g) {
            out.b[g].x = pack_bf16x2(v[g][0], v[g][1]);
            out.b[g].y = pack_bf16x2(v[g][2], v[g][3]);
        }
    } else {
#pragma unroll
        for (int g = 0; g < 32; ++g) out.v[g] = v[g];
    }
}

template <bool BF16MMA>
__device__ __forceinline__ void contract_w(uint4 w0, uint4 w1, const XM<BF16MMA> &xm, const void *__restrict__ lut,
                                           f32x4 (&acc)[32]) {
    const uint32_t wb[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int g = 0; g < 32; ++g) {
        const uint32_t byte = (wb[g >> 2] >> (8 * (g & 3))) & 0xffu;
        if constexpr (BF16MMA) {
            const uint2 wa = ((const uint2 *)lut)[byte];
            acc[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, wa),
                                                                __builtin_bit_cast(i16x4, xm.b[g]), acc[g], 0, 0, 0);
        } else {
            const f32x4 wa = ((const f32x4 *)lut)[byte];
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[s], xm.v[g][s], acc[g], 0, 0, 0);
        }
        if ((g & 7) == 7) __builtin_amdgcn_sched_barrier(0);
    }
}

// The lane's 32 code bytes of weight tile (nt, c).
__device__ __forceinline__ void load_w(const HadArgs &a, int nt, int c, int lane, uint4 &w0, uint4 &w1) {
    const uint4 *src = (const uint4 *)(a.kw + (((int64_t)nt * a.Kc + c) * 64 + lane) * 32);
    w0 = src[0];
    w1 = src[1];
}

template <bool BF16MMA>
__device__ __forceinline__ void contract(const HadArgs &a, int nt, int c, int lane, const XM<BF16MMA> &xm,
                                         const void *__restrict__ lut, f32x4 (&acc)[32]) {
    uint4 w0, w1;
    load_w(a, nt, c, lane, w0, w1);
    contract_w<BF16MMA>(w0, w1, xm, lut, acc);
}

// Output transform of a 16x16 tile (skipped with FHT = false when the caller
// has already transformed acc), beta (and RoPE) and the stores.
template <typename T, bool VEC, bool FHT = true>
__device__ __forceinline__ void transform_store(const HadArgs &a, f32x4 (&acc)[32], __amdgpu_buffer_rsrc_t yr,
                                                uint32_t row_off, bool row_ok, int nt, int q,
                                                const f32x4 *__restrict__ beta_l, int row) {
    constexpr uint32_t esz = sizeof(T);
    if constexpr (FHT) fht32x4(acc);
    const int o0 = kNTile * nt + 4 * q;
    const uint32_t hstride = (uint32_t)a.gsy * esz;
    const f32x4 *bl = beta_l + (nt * 4 + q) * 32;
    if (VEC) {
        const bool ok = row_ok && o0 < a.out_o;
        const uint32_t voff = ok ? row_off + (uint32_t)o0 * esz : kOOB;
        if (a.rope) {
            // the same two (cos, sin) pairs for all 32 groups of the row
            const f32x4 cs = ok ? rope_cs(a, row, o0) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int h = 0; h < 32; ++h) {
                Buf4<T>::store(rope_apply(acc[h] * bl[h], cs), yr, voff, (uint32_t)h * hstride);
                if ((h & 7) == 7) __builtin_amdgcn_sched_barrier(0);
            }
        } else {
#pragma unroll
            for (int h = 0; h < 32; ++h) {
                Buf4<T>::store(acc[h] * bl[h], yr, voff, (uint32_t)h * hstride);
                if ((h & 7) == 7) __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        uint32_t voff[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) voff[j] = (row_ok && o0 + j < a.out_o) ? row_off + (uint32_t)(o0 + j) * esz : kOOB;
#pragma unroll
        for (int h = 0; h < 32; ++h) {
            const f32x4 r = acc[h] * bl[h];
#pragma unroll
            for (int j = 0; j < 4; ++j) Buf4<T>::store1(r[j], yr, voff[j], (uint32_t)h * hstride);
            if ((h & 7) == 7) __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <bool BF16MMA> constexpr int dense_frag_bytes() { return BF16MMA ? 8 : 16; }

template <bool BF16MMA>
__device__ __forceinline__ void contract_dense(const unsigned char *__restrict__ wf, const XM<BF16MMA> &xm,
                                               f32x4 (&acc)[32]) {
#pragma unroll
    for (int g = 0; g < 32; ++g) {
        if constexpr (BF16MMA) {
            const uint2 wa = ((const uint2 *)wf)[g * 64];
            acc[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, wa),
                                                                __builtin_bit_cast(i16x4, xm.b[g]), acc[g], 0, 0, 0);
        } else {
            const f32x4 wa = ((const f32x4 *)wf)[g * 64];
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[s], xm.v[g][s], acc[g], 0, 0, 0);
        }
        if ((g & 7) == 7) __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace walsh
