// Hadamard-32 ternary linear forward (HadamardLinear.forward,
// src/model/fht_cuda.py:489-519), one fused kernel:
//
//   x row [32 g][in_o i]  --alpha-->  FHT over g  --W_g (ternary, per group)-->
//   FHT over g  --beta/32-->  y row [32 h][out_o o]
//
// Work split.  A wavefront owns a tile of 16 tokens.  Lane l = (t, q) with
// t = l % 16 the token and q = l / 16 a quad of columns: for a K-chunk c it
// loads x[t, g*in_o + 16c + 4q .. +3] for all 32 groups g, so both Hadamard
// transforms run entirely inside the lane's registers (5 butterfly stages on
// 32 values, no cross-lane traffic).  The per-group contraction
// y_g[o, t] = sum_i W[g, o, i] xm[t, g, i] is a 16x16 matrix-core product per
// group with A = W_g (o x i, 2-bit codes expanded through an LDS table) and
// B = xm^T (i x t, already in the lane layout the instruction wants), so the
// result lands as 4 consecutive outputs o per lane per group, ready for the
// output transform and 8/16-byte stores.
//
// Both transforms are left unnormalised; the 1/sqrt(32)^2 = 1/32 is folded
// into beta (exact: a power of two).
#include <type_traits>

#include "hadamard_core.h"

namespace walsh {

// ---------------------------------------------------------------- weights

// Kernel weight layout: [Nt][Kc][64 lanes][32 groups] bytes.  Lane l of tile
// (nt, c) holds, for each group g, the packed byte with codes
// W[g, 16nt + l%16, 16c + 4(l/16) .. +3]; that is exactly one byte of the
// reference packing (4 codes per byte along K), so the layout is a byte
// permutation.  Rows/columns past out_o/in_o hold 0x55 (four zero codes).
__global__ void hadamard_prepare_kernel(const uint8_t *__restrict__ packed, int in_o, int out_o, int Nt,
                                        int Kc, uint8_t *__restrict__ kw) {
    const int64_t total = (int64_t)Nt * Kc * 64 * 32;
    const int kp4 = (int)ceil_div(in_o, 4);
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int g = (int)(e & 31);
        const int lane = (int)((e >> 5) & 63);
        const int64_t tc = e >> 11;
        const int c = (int)(tc % Kc);
        const int nt = (int)(tc / Kc);
        const int o = kNTile * nt + (lane & 15);
        const int i0 = kKChunk * c + 4 * (lane >> 4);
        uint8_t b = 0x55;
        if (o < out_o && i0 < in_o) b = packed[((int64_t)g * out_o + o) * kp4 + i0 / 4];
        kw[e] = b;
    }
}

// VEC: in_o % 4 == 0 and out_o % 4 == 0 with aligned rows (4-wide loads and
// stores).  KC1: a single input chunk (in_o <= 16); the transformed inputs
// are computed once per tile and reused for every output tile.
// DENSE: float weights instead of ternary codes (the Hadamard head mixer),
// as matrix-core A fragments [Nt][Kc][32 g][64 lanes] (bf16x4 or f32x4)
// copied into LDS in place of the code table.
// Per-wave LDS area of the STAGED variant: the tile's 16 rows of 1 KB at a
// pitch of 1 KB + 16 bytes (16-byte aligned rows for the whole-row
// accesses).  The 8-byte fragment accesses (row t, bytes 32 g + 8 q) then
// meet rows t and t + 8 on the same banks; an 8-byte pad halves the
// bank-conflict cycles but leaves odd rows 8-byte aligned, and the kernel
// ran 6% slower with it.
constexpr int kStagePitch = 1024 + 16;
constexpr size_t kStageBytes = (size_t)kTile * kStagePitch;
// Output size of one launch from which the STAGED variant stores
// non-temporally: half the 256 MB Infinity Cache.  At 262,144 rows (256 MB
// out) that takes one layer from 117 us to 102 us.
constexpr int64_t kStreamOutBytes = (int64_t)128 << 20;

// PIPE1: the bf16 single-chunk, single-output-tile shape (in_o, out_o <= 16,
// VEC, not DENSE) in its own software-pipelined loop.
// STAGED (with PIPE1): rows of exactly 512 contiguous bf16 on both sides
// (in_o = out_o = gsx = gsy = 16, ldx = ldy = 512, plain rows).  Each wave
// moves its tile as 16 whole 1 KB rows, 16 bytes per lane, through its own
// LDS area (kStageRows rows at kStagePitch bytes) instead of loading and
// storing 32-byte row segments per lane quad: the segment pattern alone
// (16 rows x 32 bytes per instruction) holds a copy kernel to about half of
// what whole-row accesses reach.  The arithmetic is PIPE1's, so the results
// are equal bitwise.
template <typename T, bool BF16MMA, bool VEC, bool KC1, bool DENSE, bool PIPE1 = false, bool STAGED = false>
__device__ __forceinline__ void hadamard_fwd_body(const HadArgs &a, int blk, int nblk) {
    static_assert(!PIPE1 || (BF16MMA && VEC && KC1 && !DENSE), "PIPE1 shape");
    static_assert(!STAGED || PIPE1, "STAGED is a PIPE1 variant");
    extern __shared__ __align__(16) unsigned char smem[];
    void *lut = smem;
    const size_t wbytes = DENSE ? (size_t)a.Nt * a.Kc * 32 * 64 * dense_frag_bytes<BF16MMA>() : lut_bytes<BF16MMA>();
    f32x4 *alpha_l = (f32x4 *)(smem + wbytes);
    f32x4 *beta_l = alpha_l + a.Kc * 128;

    const int tid = threadIdx.x;
    if constexpr (DENSE) {
        const uint4 *src = (const uint4 *)a.kw;
        for (int e = tid; e < (int)(wbytes / 16); e += kThreads) ((uint4 *)smem)[e] = src[e];
    } else {
        const uint32_t byte = (uint32_t)tid;  // kThreads == 256 table entries
        float val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) val[j] = (float)((int)((byte >> (6 - 2 * j)) & 3u) - 1);
        if constexpr (BF16MMA) {
            uint2 e;
            e.x = pack_bf16x2(val[0], val[1]);
            e.y = pack_bf16x2(val[2], val[3]);
            ((uint2 *)lut)[byte] = e;
        } else {
            ((f32x4 *)lut)[byte] = f32x4{val[0], val[1], val[2], val[3]};
        }
    }
    for (int e = tid; e < a.Kc * 128; e += kThreads) {  // e = (c*4 + q)*32 + g
        const int g = e & 31, cq = e >> 5;
        const int i0 = 4 * cq;  // 16c + 4q
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = (i0 + j < a.in_o) ? (a.alpha ? a.alpha[g * a.in_o + i0 + j] : 1.f) : 0.f;
        alpha_l[e] = v;
    }
    for (int e = tid; e < a.Nt * 128; e += kThreads) {
        const int h = e & 31, nq = e >> 5;
        const int o0 = 4 * nq;
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (o0 + j < a.out_o) ? a.beta[h * a.beta_h + o0 + j] * 0.03125f : 0.f;
        beta_l[e] = v;
    }
    __syncthreads();

    constexpr uint32_t esz = sizeof(T);
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int t = lane & 15;
    const int q = lane >> 4;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a, esz));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * esz));
    const int n_tiles = (int)ceil_div(a.M, kTile);
    const int wt = a.wave_tiles > 0 ? a.wave_tiles : kWaves;
    if (wave >= wt) return;   // after the set-up barrier; the tile loop has none
    const int stride = nblk * wt;
    auto contract_any = [&](int nt, int c, const XM<BF16MMA> &xm, f32x4 (&acc)[32]) {
        if constexpr (DENSE)
            contract_dense<BF16MMA>(smem + ((size_t)(nt * a.Kc + c) * 32 * 64 + lane) * dense_frag_bytes<BF16MMA>(),
                                    xm, acc);
        else
            contract<BF16MMA>(a, nt, c, lane, xm, lut, acc);
    };

    if constexpr (PIPE1) {
        // bf16, one input chunk and one output tile (in_o, out_o <= 16):
        // software-pipelined over the wave's tiles.
        // The next tile's x (raw bf16, 64 registers) is requested right after
        // the last products of the current one, so its loads are in flight
        // during the output transform and the stores; the input transform
        // runs in two passes of 2 columns (64 registers of float pairs).
        const int i0 = 4 * q;
        const uint32_t gsb = (uint32_t)a.gsx * 2;
        auto x_off = [&](int tl) -> uint32_t {
            const int r = tl * kTile + t;
            return (tl < n_tiles && r < a.M && i0 < a.in_o) ? x_row_off(a, r, 2) + (uint32_t)i0 * 2 : kOOB;
        };
        const f32x4 *al = alpha_l + q * 32;
        u32x2 xraw[32];
        int tile = blk * wt + wave;
        // STAGED: the tile's rows (row i of the tile in xrow[i]) and the
        // wave's LDS area
        [[maybe_unused]] u32x4 xrow[STAGED ? kTile : 1];
        [[maybe_unused]] unsigned char *area = (unsigned char *)(beta_l + a.Nt * 128) + (size_t)wave * kStageBytes;
        [[maybe_unused]] auto load_rows = [&](int tl) {
#pragma unroll
            for (int i = 0; i < kTile; ++i) {
                const int r = tl * kTile + i;
                xrow[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t)lane * 16,
                                                                (tl < n_tiles && r < a.M) ? (uint32_t)r * 1024u : kOOB, 0);
            }
        };
        if constexpr (STAGED) {
            load_rows(tile);
        } else {
            const uint32_t o0 = x_off(tile);
#pragma unroll
            for (int g = 0; g < 32; ++g) xraw[g] = __builtin_amdgcn_raw_buffer_load_b64(xr, o0, (uint32_t)g * gsb, 0);
        }
        for (; tile < n_tiles; tile += stride) {
            if constexpr (STAGED) {
                // rows into the area, then each lane's 8 bytes of the 32
                // groups of row t (the wave's LDS operations run in order;
                // the fences keep the compiler from moving them)
#pragma unroll
                for (int i = 0; i < kTile; ++i) *(u32x4 *)(area + i * kStagePitch + lane * 16) = xrow[i];
                wave_lds_fence();
#pragma unroll
                for (int g = 0; g < 32; ++g) xraw[g] = *(const u32x2 *)(area + t * kStagePitch + g * 32 + q * 8);
                wave_lds_fence();
            }
            const int row = tile * kTile + t;
            const bool row_ok = row < a.M;
            const uint32_t yoff = (uint32_t)((int64_t)row * a.ldy * esz);
            XM<true> xm;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                f32x2 v[32];
#pragma unroll
                for (int g = 0; g < 32; ++g) {
                    const uint32_t u = p ? xraw[g].y : xraw[g].x;
                    const f32x2 ag = *((const f32x2 *)&al[g] + p);
                    v[g] = f32x2{__uint_as_float(u << 16) * ag[0], __uint_as_float(u & 0xffff0000u) * ag[1]};
                    if ((g & 7) == 7) __builtin_amdgcn_sched_barrier(0);
                }
                fht32<f32x2>(v);
#pragma unroll
                for (int g = 0; g < 32; ++g) ((uint32_t *)&xm.b[g])[p] = pack_bf16x2(v[g][0], v[g][1]);
            }
            {
                constexpr int nt = 0;
                f32x4 acc[32];
#pragma unroll
                for (int g = 0; g < 32; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
                contract<true>(a, nt, 0, lane, xm, lut, acc);
                // the next tile's x is requested before any store of this one:
                // a wait for a load also waits for every memory operation
                // issued before it, so loads queued behind stores would wait
                // for the stores
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (STAGED) {
                    load_rows(tile + stride);
                } else {
                    const uint32_t on = x_off(tile + stride);
#pragma unroll
                    for (int g = 0; g < 32; ++g)
                        xraw[g] = __builtin_amdgcn_raw_buffer_load_b64(xr, on, (uint32_t)g * gsb, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
                // output transform, then beta (and RoPE) and the stores
                fht32x4(acc);
                const int o0 = kNTile * nt + 4 * q;
                const bool ok = row_ok && o0 < a.out_o;
                const uint32_t voff = ok ? yoff + (uint32_t)o0 * 2 : kOOB;
                const uint32_t hstride = (uint32_t)a.gsy * 2;
                const f32x4 *bl = beta_l + (nt * 4 + q) * 32;
                const bool rope = a.rope != nullptr;
                const f32x4 cs = (rope && ok) ? rope_cs(a, row, o0) : f32x4{1.f, 0.f, 1.f, 0.f};
                auto stores = [&](auto with_rope) {
#pragma unroll
                    for (int h0 = 0; h0 < 32; h0 += 4) {
                        f32x4 b8[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j) b8[j] = bl[h0 + j];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            f32x4 r = acc[h0 + j] * b8[j];
                            if constexpr (decltype(with_rope)::value) r = rope_apply(r, cs);
                            if constexpr (STAGED) {
                                u32x2 u;
                                u.x = pack_bf16x2(r.x, r.y);
                                u.y = pack_bf16x2(r.z, r.w);
                                *(u32x2 *)(area + t * kStagePitch + (h0 + j) * 32 + q * 8) = u;
                            } else {
                                Buf4<uint16_t>::store(r, yr, voff, (uint32_t)(h0 + j) * hstride);
                            }
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                };
                if (rope) stores(std::true_type{});
                else stores(std::false_type{});
                if constexpr (STAGED) {
                    // whole output rows out of the area (rows past M fall
                    // outside the buffer and are dropped)
                    wave_lds_fence();
                    auto store_rows = [&](auto aux) {
#pragma unroll
                        for (int i = 0; i < kTile; ++i) {
                            const u32x4 v = *(const u32x4 *)(area + i * kStagePitch + lane * 16);
                            __builtin_amdgcn_raw_buffer_store_b128(v, yr, (uint32_t)lane * 16,
                                                                   (uint32_t)(tile * kTile + i) * 1024u,
                                                                   decltype(aux)::value);
                        }
                    };
                    // cache policy 2: non-temporal
                    if (a.nt_store) store_rows(std::integral_constant<int, 2>{});
                    else store_rows(std::integral_constant<int, 0>{});
                    wave_lds_fence();
                }
            }
        }
        return;
    }
    for (int tile = blk * wt + wave; tile < n_tiles; tile += stride) {
        const int row = tile * kTile + t;
        const bool row_ok = row < a.M;
        const uint32_t xoff = row_ok ? x_row_off(a, row, esz) : 0u;
        const uint32_t yoff = (uint32_t)((int64_t)row * a.ldy * esz);
        if constexpr (KC1) {
            XM<BF16MMA> xm;
            load_transform<T, BF16MMA, VEC>(a, xr, xoff, row_ok, 0, q, alpha_l, xm);
            for (int nt = 0; nt < a.Nt; ++nt) {
                f32x4 acc[32];
#pragma unroll
                for (int g = 0; g < 32; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
                contract_any(nt, 0, xm, acc);
                transform_store<T, VEC>(a, acc, yr, yoff, row_ok, nt, q, beta_l, row);
            }
        } else {
            for (int nt = 0; nt < a.Nt; ++nt) {
                f32x4 acc[32];
#pragma unroll
                for (int g = 0; g < 32; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int c = 0; c < a.Kc; ++c) {
                    XM<BF16MMA> xm;
                    load_transform<T, BF16MMA, VEC>(a, xr, xoff, row_ok, c, q, alpha_l, xm);
                    contract_any(nt, c, xm, acc);
                }
                transform_store<T, VEC>(a, acc, yr, yoff, row_ok, nt, q, beta_l, row);
            }
        }
    }
}

template <typename T, bool BF16MMA, bool VEC, bool KC1, bool DENSE = false, bool PIPE1 = false, bool STAGED = false>
__global__ __launch_bounds__(kThreads, (BF16MMA && KC1 && VEC) ? 2 : 1) void hadamard_fwd_kernel(HadArgs a) {
    hadamard_fwd_body<T, BF16MMA, VEC, KC1, DENSE, PIPE1, STAGED>(a, blockIdx.x, gridDim.x);
}

// Several Hadamard linears of one shape on the same input rows in one launch
// (the q, k and v projections): workgroup b runs layer b % n over the tiles
// of slot b / n, so the n layers' waves fill the machine together and the
// shared input is fetched from HBM once (later reads hit the caches).
constexpr int kMaxMulti = 4;
struct HadArgsN {
    HadArgs p[kMaxMulti];
    int n;
};

template <typename T, bool BF16MMA, bool VEC, bool KC1, bool PIPE1 = false, bool STAGED = false>
__global__ __launch_bounds__(kThreads, (BF16MMA && KC1 && VEC) ? 2 : 1) void hadamard_fwdn_kernel(HadArgsN an) {
    const int l = blockIdx.x % an.n;
    hadamard_fwd_body<T, BF16MMA, VEC, KC1, false, PIPE1, STAGED>(an.p[l], blockIdx.x / an.n, gridDim.x / an.n);
}

// ---------------------------------------------------------------- wavefront pairs
// bf16, in_o <= 16 and out_o <= 16 (one input chunk, one output tile), VEC
// layouts: the PIPE1 shape with each 16-token tile split over a PAIR of
// wavefronts by group, so a wavefront holds 16 groups (half the registers
// and half the dependent chain of the one-wavefront kernel; twice the
// wavefronts in flight).  Every butterfly of both transforms is computed as
// in fht32 (stages h = 1, 2, 4, 8, 16 in that order, (a, b) -> (a + b, a - b)
// with a the lower group), so results equal hadamard_fwd_kernel's bitwise.
//
// Wavefront HF of the pair loads groups 16 HF .. 16 HF + 15 (slot s = group
// - 16 HF) and runs input stages 1..8 locally.  Stage 16 pairs group g with
// g + 16 across the pair: HF 0 computes the pairs g = 0..7, HF 1 the pairs
// g = 8..15, each sending the other the 8 slots it needs (8 KB through LDS)
// and keeping both results of its pairs, so afterwards slot s holds group
//   g_in(s) = 8 HF + (s & 7) + 16 (s >> 3).
// The contraction runs on those 16 groups.  Output stages 1, 2, 4 pair slots
// within (s & 7); stage 8 pairs g_in(s) with g_in(s) + 8 across the pair (HF 0
// computes the pairs with s & 4 == 0, HF 1 those with s & 4 != 0; low result
// to the slot with bit 2 clear, high to the one with bit 2 set), after which
// slot u holds group
//   g_out(u) = (u & 3) + 4 HF + 8 ((u >> 2) & 1) + 16 (u >> 3),
// and stage 16 pairs slots u and u + 8 locally.
// Several layers on the same input rows (q, k, v): workgroup b runs layer
// b % n over tiles b / n, b / n + G / n, ... as hadamard_fwdn_kernel does.
constexpr int kPairThreads = 128;
// Above this many 16-row tiles per layer the one-wavefront kernel (its next
// tile's loads in flight during the current one's output) is faster once the
// rows come from HBM rather than the Infinity Cache: 65,536 bf16 rows from
// buffers rotated past the cache take 48.7 us here against 44.1 us there,
// while at 8,192 rows one layer takes 9.8 us against 14.2 us and q, k, v
// 19.1 us against 23.8 us.
constexpr int64_t kPairMaxTiles = 2048;
// Where the one-wavefront kernel moves whole 1 KB rows through LDS (the
// STAGED variant: 16x16 layers on contiguous rows) it is faster from fewer
// tiles on: at 32,768 rows one layer takes 21.3 us against the pairs'
// 22.7 us (20.9 against 22.8 from HBM), at 16,384 rows 16.1 against 15.0.
constexpr int64_t kPairMaxTilesRows = 1024;
constexpr size_t kPairLds = 256 * 8 + 2 * 128 * 16 + 2 * 8 * 64 * 16;   // lut, alpha/beta, exchange

template <int HF, bool DENSE>
__device__ __forceinline__ void pair_tile(const HadArgs &a, int tile, int lane, const uint2 *__restrict__ lut,
                                          const f32x4 *__restrict__ alpha_l, const f32x4 *__restrict__ beta_l,
                                          f32x4 *__restrict__ xch, __amdgpu_buffer_rsrc_t xr,
                                          __amdgpu_buffer_rsrc_t yr) {
    const int t = lane & 15, q = lane >> 4;
    const int row = tile * kTile + t;
    const bool row_ok = row < a.M;
    f32x4 *mine = xch + HF * 8 * 64, *theirs = xch + (1 - HF) * 8 * 64;
    // the lane's 32 code bytes (issued first: their wait is after the input
    // transform); DENSE reads its weight fragments just before the products
    uint4 w0, w1;
    if constexpr (!DENSE) load_w(a, 0, 0, lane, w0, w1);
    // input: groups 16 HF + s, columns 4q .. 4q + 3
    f32x4 v[16];
    {
        const uint32_t gsb = (uint32_t)a.gsx * 2;
        const uint32_t xo = (row_ok && 4 * q < a.in_o) ? x_row_off(a, row, 2) + (uint32_t)(8 * q) : kOOB;
        u32x2 xraw[16];
#pragma unroll
        for (int s = 0; s < 16; ++s)
            xraw[s] = __builtin_amdgcn_raw_buffer_load_b64(xr, xo, (uint32_t)(16 * HF + s) * gsb, 0);
        const f32x4 *al = alpha_l + q * 32 + 16 * HF;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const f32x4 x4 = {__uint_as_float(xraw[s].x << 16), __uint_as_float(xraw[s].x & 0xffff0000u),
                              __uint_as_float(xraw[s].y << 16), __uint_as_float(xraw[s].y & 0xffff0000u)};
            v[s] = x4 * al[s];
        }
    }
#pragma unroll
    for (int h = 1; h < 16; h <<= 1) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            if (s & h) continue;
            const f32x4 x0 = v[s], x1 = v[s + h];
            v[s] = x0 + x1;
            v[s + h] = x0 - x1;
        }
    }
    // input stage 16 across the pair
    lds_barrier();   // the partner is done reading the previous tile's output exchange
#pragma unroll
    for (int j = 0; j < 8; ++j) mine[j * 64 + lane] = v[HF ? j : j + 8];
    lds_barrier();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const f32x4 other = theirs[j * 64 + lane];
        if (HF == 0) {
            const f32x4 x0 = v[j], x1 = other;           // groups j, 16 + j
            v[j] = x0 + x1;
            v[j + 8] = x0 - x1;
        } else {
            const f32x4 x0 = other, x1 = v[j + 8];       // groups 8 + j, 24 + j
            v[j] = x0 + x1;
            v[j + 8] = x0 - x1;
        }
    }
    // contraction of the 16 groups g_in(s)
    u32x2 xm[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) xm[s] = u32x2{pack_bf16x2(v[s].x, v[s].y), pack_bf16x2(v[s].z, v[s].w)};
    uint2 wd[16];
    if constexpr (DENSE) {
        const uint2 *wf = (const uint2 *)a.kw;   // [32 g][64 lanes] bf16x4
#pragma unroll
        for (int s = 0; s < 16; ++s) wd[s] = wf[(8 * HF + (s & 7) + 16 * (s >> 3)) * 64 + lane];
    }
    f32x4 acc[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        uint2 wa;
        if constexpr (DENSE) {
            wa = wd[s];
        } else {
            const uint32_t wb[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            const int g = 8 * HF + (s & 7) + 16 * (s >> 3);
            wa = lut[(wb[g >> 2] >> (8 * (g & 3))) & 0xffu];
        }
        acc[s] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, wa),
                                                            __builtin_bit_cast(i16x4, xm[s]),
                                                            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    }
    // output stages 1, 2, 4 within (s & 7)
#pragma unroll
    for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            if (s & h) continue;
            const f32x4 x0 = acc[s], x1 = acc[s + h];
            acc[s] = x0 + x1;
            acc[s + h] = x0 - x1;
        }
    }
    // output stage 8 across the pair: HF keeps slots with (s & 4) == 4 HF
    lds_barrier();   // the partner is done reading the input exchange
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int snd = (p & 3) + 4 * (1 - HF) + 8 * (p >> 2);
        mine[p * 64 + lane] = acc[snd];
    }
    lds_barrier();
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int kept = (p & 3) + 4 * HF + 8 * (p >> 2);
        const int lo = kept & ~4, hi = kept | 4;
        const f32x4 other = theirs[p * 64 + lane];
        const f32x4 x0 = HF == 0 ? acc[kept] : other;   // group with bit 3 clear
        const f32x4 x1 = HF == 0 ? other : acc[kept];   // its partner + 8
        acc[lo] = x0 + x1;
        acc[hi] = x0 - x1;
    }
    // output stage 16: slots u, u + 8
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const f32x4 x0 = acc[u], x1 = acc[u + 8];
        acc[u] = x0 + x1;
        acc[u + 8] = x0 - x1;
    }
    // beta (and RoPE), stores of groups g_out(u)
    const int o0 = 4 * q;
    const bool ok = row_ok && o0 < a.out_o;
    const uint32_t voff = ok ? (uint32_t)((int64_t)row * a.ldy * 2) + (uint32_t)o0 * 2 : kOOB;
    const uint32_t hstride = (uint32_t)a.gsy * 2;
    const f32x4 *bl = beta_l + q * 32;
    if (a.rope) {
        const f32x4 cs = ok ? rope_cs(a, row, o0) : f32x4{1.f, 0.f, 1.f, 0.f};
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int h = (u & 3) + 4 * HF + 8 * ((u >> 2) & 1) + 16 * (u >> 3);
            Buf4<uint16_t>::store(rope_apply(acc[u] * bl[h], cs), yr, voff, (uint32_t)h * hstride);
        }
    } else {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int h = (u & 3) + 4 * HF + 8 * ((u >> 2) & 1) + 16 * (u >> 3);
            Buf4<uint16_t>::store(acc[u] * bl[h], yr, voff, (uint32_t)h * hstride);
        }
    }
}

// ---------------------------------------------------------------- head mixer + output projection
// The attention block's head mixer (dense per-head weights, head_dim 16) and
// the output projection (a 16x16 ternary Hadamard linear) on the same rows in
// one launch, on wavefront pairs: the mixer's tile is computed as
// hadamard_pair_kernel<true> computes it, rounded to bf16 as its store would
// round it, handed to the projection's input layout through LDS and run
// through the projection as hadamard_pair_kernel<false> runs it, so the
// output equals the two launches' bitwise without the intermediate rows
// going through memory.

// Input transform (stages 1..8 local, 16 across the pair), the contraction of
// groups g_in(s) and the output transform of pair_tile: v holds the scaled
// inputs of groups 16 HF + s; on return acc[u] holds group g_out(u) before
// beta.
template <int HF, bool DENSE>
__device__ __forceinline__ void pair_core(const HadArgs &a, int lane, const uint2 *__restrict__ lut, f32x4 *xch,
                                          uint4 w0, uint4 w1, f32x4 (&v)[16], f32x4 (&acc)[16]) {
    f32x4 *mine = xch + HF * 8 * 64, *theirs = xch + (1 - HF) * 8 * 64;
#pragma unroll
    for (int h = 1; h < 16; h <<= 1) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            if (s & h) continue;
            const f32x4 x0 = v[s], x1 = v[s + h];
            v[s] = x0 + x1;
            v[s + h] = x0 - x1;
        }
    }
    lds_barrier();   // the partner is done reading the previous exchange
#pragma unroll
    for (int j = 0; j < 8; ++j) mine[j * 64 + lane] = v[HF ? j : j + 8];
    lds_barrier();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const f32x4 other = theirs[j * 64 + lane];
        if (HF == 0) {
            const f32x4 x0 = v[j], x1 = other;
            v[j] = x0 + x1;
            v[j + 8] = x0 - x1;
        } else {
            const f32x4 x0 = other, x1 = v[j + 8];
            v[j] = x0 + x1;
            v[j + 8] = x0 - x1;
        }
    }
    u32x2 xm[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) xm[s] = u32x2{pack_bf16x2(v[s].x, v[s].y), pack_bf16x2(v[s].z, v[s].w)};
    uint2 wd[16];
    if constexpr (DENSE) {
        const uint2 *wf = (const uint2 *)a.kw;   // [32 g][64 lanes] bf16x4
#pragma unroll
        for (int s = 0; s < 16; ++s) wd[s] = wf[(8 * HF + (s & 7) + 16 * (s >> 3)) * 64 + lane];
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        uint2 wa;
        if constexpr (DENSE) {
            wa = wd[s];
        } else {
            const uint32_t wb[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            const int g = 8 * HF + (s & 7) + 16 * (s >> 3);
            wa = lut[(wb[g >> 2] >> (8 * (g & 3))) & 0xffu];
        }
        acc[s] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, wa),
                                                            __builtin_bit_cast(i16x4, xm[s]),
                                                            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    }
#pragma unroll
    for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            if (s & h) continue;
            const f32x4 x0 = acc[s], x1 = acc[s + h];
            acc[s] = x0 + x1;
            acc[s + h] = x0 - x1;
        }
    }
    lds_barrier();   // the partner is done reading the input exchange
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int snd = (p & 3) + 4 * (1 - HF) + 8 * (p >> 2);
        mine[p * 64 + lane] = acc[snd];
    }
    lds_barrier();
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int kept = (p & 3) + 4 * HF + 8 * (p >> 2);
        const int lo = kept & ~4, hi = kept | 4;
        const f32x4 other = theirs[p * 64 + lane];
        const f32x4 x0 = HF == 0 ? acc[kept] : other;
        const f32x4 x1 = HF == 0 ? other : acc[kept];
        acc[lo] = x0 + x1;
        acc[hi] = x0 - x1;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const f32x4 x0 = acc[u], x1 = acc[u + 8];
        acc[u] = x0 + x1;
        acc[u + 8] = x0 - x1;
    }
}

template <int HF>
__device__ __forceinline__ void mixproj_tile(const HadArgs &m, const HadArgs &p, int tile, int lane,
                                             const uint2 *__restrict__ lut, const f32x4 *__restrict__ mbeta_l,
                                             const f32x4 *__restrict__ palpha_l, const f32x4 *__restrict__ pbeta_l,
                                             f32x4 *xch, __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t yr) {
    const int t = lane & 15, q = lane >> 4;
    const int row = tile * kTile + t;
    const bool row_ok = row < m.M;
    f32x4 *mine = xch + HF * 8 * 64, *theirs = xch + (1 - HF) * 8 * 64;
    uint4 w0, w1;
    f32x4 v[16], acc[16];
    {
        // the mixer's input: heads 16 HF + s of the row (its alpha is 1)
        const uint32_t gsb = (uint32_t)m.gsx * 2;
        const uint32_t xo = row_ok ? x_row_off(m, row, 2) + (uint32_t)(8 * q) : kOOB;
        u32x2 xraw[16];
#pragma unroll
        for (int s = 0; s < 16; ++s)
            xraw[s] = __builtin_amdgcn_raw_buffer_load_b64(xr, xo, (uint32_t)(16 * HF + s) * gsb, 0);
#pragma unroll
        for (int s = 0; s < 16; ++s)
            v[s] = f32x4{__uint_as_float(xraw[s].x << 16), __uint_as_float(xraw[s].x & 0xffff0000u),
                         __uint_as_float(xraw[s].y << 16), __uint_as_float(xraw[s].y & 0xffff0000u)};
    }
    pair_core<HF, true>(m, lane, lut, xch, w0, w1, v, acc);
    // the projection's code bytes (requested here: live through the mixer
    // they would push the kernel past its register budget)
    load_w(p, 0, 0, lane, w0, w1);
    // the mixer's beta and bf16 rounding: slot u holds group g_out(u)
    const f32x4 *mb = mbeta_l + q * 32;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int h = (u & 3) + 4 * HF + 8 * ((u >> 2) & 1) + 16 * (u >> 3);
        const f32x4 r = acc[u] * mb[h];
        const uint32_t lo = pack_bf16x2(r.x, r.y), hi = pack_bf16x2(r.z, r.w);
        acc[u] = f32x4{__uint_as_float(lo << 16), __uint_as_float(lo & 0xffff0000u), __uint_as_float(hi << 16),
                       __uint_as_float(hi & 0xffff0000u)};
    }
    // to the projection's layout (groups 16 HF + s): slots u >> 3 == HF hold
    // groups of this half, the others go to the partner
    lds_barrier();   // the partner is done reading the output exchange
#pragma unroll
    for (int j = 0; j < 8; ++j) mine[j * 64 + lane] = acc[8 * (1 - HF) + j];
    lds_barrier();
    const f32x4 *pa = palpha_l + q * 32 + 16 * HF;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int own = (j & 3) + 4 * HF + 8 * ((j >> 2) & 1);
        const int other = (j & 3) + 4 * (1 - HF) + 8 * ((j >> 2) & 1);
        v[own] = acc[8 * HF + j] * pa[own];
        v[other] = theirs[j * 64 + lane] * pa[other];
    }
    pair_core<HF, false>(p, lane, lut, xch, w0, w1, v, acc);
    // the projection's beta and the stores of groups g_out(u)
    const int o0 = 4 * q;
    const uint32_t voff = row_ok ? (uint32_t)((int64_t)row * p.ldy * 2) + (uint32_t)o0 * 2 : kOOB;
    const uint32_t hstride = (uint32_t)p.gsy * 2;
    const f32x4 *pb = pbeta_l + q * 32;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int h = (u & 3) + 4 * HF + 8 * ((u >> 2) & 1) + 16 * (u >> 3);
        Buf4<uint16_t>::store(acc[u] * pb[h], yr, voff, (uint32_t)h * hstride);
    }
}

constexpr size_t kMixProjLds = 256 * 8 + 3 * 128 * 16 + 2 * 8 * 64 * 16;   // lut, 3 tables, exchange

// m: the mixer (HadArgs of walsh_head_mixer_fwd), p: the projection (in_o =
// out_o = 16, its x unused: the mixer's output rows).
__global__ __launch_bounds__(kPairThreads, 2) void hadamard_pair_mixproj_kernel(HadArgs m, HadArgs p) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint2 *lut = (uint2 *)smem;
    f32x4 *mbeta_l = (f32x4 *)(smem + 256 * 8);   // [4 q][32 h]
    f32x4 *palpha_l = mbeta_l + 128;               // [4 q][32 g]
    f32x4 *pbeta_l = palpha_l + 128;               // [4 q][32 h]
    f32x4 *xch = pbeta_l + 128;                    // [2 HF][8][64 lanes]
    const int tid = threadIdx.x;
    for (int e = tid; e < 256; e += kPairThreads) {
        float val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) val[j] = (float)((int)(((uint32_t)e >> (6 - 2 * j)) & 3u) - 1);
        lut[e] = uint2{pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3])};
    }
    {
        const int e = tid;   // (q, g) = (e >> 5, e & 31); kPairThreads == 128 entries
        const int g = e & 31, i0 = 4 * (e >> 5);
        // buffer loads issued together, with no branch around them (no
        // alpha: a resource of no records), converted after
        const __amdgpu_buffer_rsrc_t mbr = make_rsrc(m.beta, (uint32_t)((31 * m.beta_h + 16) * 4));
        const __amdgpu_buffer_rsrc_t par = make_rsrc(p.alpha, p.alpha ? (uint32_t)((31 * p.in_o + 16) * 4) : 0u);
        const __amdgpu_buffer_rsrc_t pbr = make_rsrc(p.beta, (uint32_t)((31 * p.beta_h + 16) * 4));
        uint32_t rm[4], ra[4], rp[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            rm[j] = __builtin_amdgcn_raw_buffer_load_b32(mbr, (uint32_t)(g * m.beta_h + i0 + j) * 4, 0, 0);
            ra[j] = __builtin_amdgcn_raw_buffer_load_b32(par, (uint32_t)(g * p.in_o + i0 + j) * 4, 0, 0);
            rp[j] = __builtin_amdgcn_raw_buffer_load_b32(pbr, (uint32_t)(g * p.beta_h + i0 + j) * 4, 0, 0);
        }
        f32x4 mb, pa, pb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mb[j] = __uint_as_float(rm[j]) * 0.03125f;
            pa[j] = p.alpha ? __uint_as_float(ra[j]) : 1.f;
            pb[j] = __uint_as_float(rp[j]) * 0.03125f;
        }
        mbeta_l[e] = mb;
        palpha_l[e] = pa;
        pbeta_l[e] = pb;
    }
    __syncthreads();
    const int hf = tid >> 6, lane = tid & 63;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(m.x, x_bytes(m, 2));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(p.y, (uint32_t)((int64_t)m.M * p.ldy * 2));
    const int n_tiles = (int)ceil_div(m.M, kTile);
    for (int tile = (int)blockIdx.x; tile < n_tiles; tile += (int)gridDim.x) {
        if (hf == 0) mixproj_tile<0>(m, p, tile, lane, lut, mbeta_l, palpha_l, pbeta_l, xch, xr, yr);
        else mixproj_tile<1>(m, p, tile, lane, lut, mbeta_l, palpha_l, pbeta_l, xch, xr, yr);
    }
}

// The pair kernel for several input chunks: bf16, 16 < in_o <= 64, out_o <= 16 (2 to 4 input chunks, one output tile),
// no RoPE: the FFN down projection at n_embd 512.  A workgroup of Kc
// wavefront pairs per 16-row tile.  Pair c loads input chunk c and runs its
// input transform and stage-16 exchange (the bulk of the dependent chain,
// now Kc-way parallel); pairs 1 .. Kc - 1 hand their packed inputs (the
// products' B operands) to pair 0 through their exchange areas; pair 0 runs the
// contraction in chunk order (one accumulator chain, as the chunk loop does),
// the output transform and the stores: results equal hadamard_fwd_kernel's
// chunk loop bitwise.  Every wavefront passes the same barriers (six per tile).
constexpr int kPairMaxKc = 4;
constexpr int kKparMaxKc = kPairMaxKc;
constexpr size_t kpar_lds(int Kc) { return 256 * 8 + (size_t)(Kc + 1) * 128 * 16 + (size_t)Kc * 2 * 8 * 64 * 16; }

template <int HF>
__device__ __forceinline__ void kpar_tile(const HadArgs &a, int tile, int pair, int lane, const uint2 *__restrict__ lut,
                                          const f32x4 *__restrict__ alpha_l, const f32x4 *__restrict__ beta_l,
                                          f32x4 *xch_all, __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t yr) {
    const int t = lane & 15, q = lane >> 4;
    const int row = tile * kTile + t;
    const bool row_ok = row < a.M;
    f32x4 *xch = xch_all + pair * 2 * 8 * 64;
    f32x4 *mine = xch + HF * 8 * 64, *theirs = xch + (1 - HF) * 8 * 64;
    const int c = pair;   // this pair's input chunk: columns 16c + 4q .. + 3
    u32x2 xm[16];
    {
        const uint32_t gsb = (uint32_t)a.gsx * 2;
        const int i0 = kKChunk * c + 4 * q;
        const uint32_t xo = (row_ok && i0 < a.in_o) ? x_row_off(a, row, 2) + (uint32_t)(2 * i0) : kOOB;
        u32x2 xraw[16];
#pragma unroll
        for (int s = 0; s < 16; ++s)
            xraw[s] = __builtin_amdgcn_raw_buffer_load_b64(xr, xo, (uint32_t)(16 * HF + s) * gsb, 0);
        const f32x4 *al = alpha_l + (c * 4 + q) * 32 + 16 * HF;
        f32x4 v[16];
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const f32x4 x4 = {__uint_as_float(xraw[s].x << 16), __uint_as_float(xraw[s].x & 0xffff0000u),
                              __uint_as_float(xraw[s].y << 16), __uint_as_float(xraw[s].y & 0xffff0000u)};
            v[s] = x4 * al[s];
        }
#pragma unroll
        for (int h = 1; h < 16; h <<= 1) {
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                if (s & h) continue;
                const f32x4 x0 = v[s], x1 = v[s + h];
                v[s] = x0 + x1;
                v[s + h] = x0 - x1;
            }
        }
        lds_barrier();   // B1: every wave is done with the previous tile's areas
#pragma unroll
        for (int j = 0; j < 8; ++j) mine[j * 64 + lane] = v[HF ? j : j + 8];
        lds_barrier();   // B2
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const f32x4 other = theirs[j * 64 + lane];
            const f32x4 x0 = HF == 0 ? v[j] : other, x1 = HF == 0 ? other : v[j + 8];
            v[j] = x0 + x1;
            v[j + 8] = x0 - x1;
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) xm[s] = u32x2{pack_bf16x2(v[s].x, v[s].y), pack_bf16x2(v[s].z, v[s].w)};
    }
    lds_barrier();   // B3: the partner has read this wave's exchange slots
    if (pair > 0) {
        u32x2 *out = (u32x2 *)mine;   // 16 slots x 64 lanes x 8 bytes: the wave's half of the area
#pragma unroll
        for (int s = 0; s < 16; ++s) out[s * 64 + lane] = xm[s];
    }
    lds_barrier();   // B4
    f32x4 acc[16];
    if (pair == 0) {
#pragma unroll
        for (int s = 0; s < 16; ++s) acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int cc = 0; cc < a.Kc; ++cc) {
            uint4 w0, w1;
            load_w(a, 0, cc, lane, w0, w1);
            u32x2 xc[16];
            if (cc == 0) {
#pragma unroll
                for (int s = 0; s < 16; ++s) xc[s] = xm[s];
            } else {
                const u32x2 *in = (const u32x2 *)(xch_all + cc * 2 * 8 * 64 + HF * 8 * 64);
#pragma unroll
                for (int s = 0; s < 16; ++s) xc[s] = in[s * 64 + lane];
            }
            const uint32_t wb[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int g = 8 * HF + (s & 7) + 16 * (s >> 3);
                acc[s] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                    __builtin_bit_cast(i16x4, lut[(wb[g >> 2] >> (8 * (g & 3))) & 0xffu]),
                    __builtin_bit_cast(i16x4, xc[s]), acc[s], 0, 0, 0);
            }
        }
#pragma unroll
        for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                if (s & h) continue;
                const f32x4 x0 = acc[s], x1 = acc[s + h];
                acc[s] = x0 + x1;
                acc[s + h] = x0 - x1;
            }
        }
    }
    lds_barrier();   // B5: pair 0's area was last read before B3
    if (pair == 0) {
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int snd = (p & 3) + 4 * (1 - HF) + 8 * (p >> 2);
            mine[p * 64 + lane] = acc[snd];
        }
    }
    lds_barrier();   // B6
    if (pair != 0) return;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int kept = (p & 3) + 4 * HF + 8 * (p >> 2);
        const int lo = kept & ~4, hi = kept | 4;
        const f32x4 other = theirs[p * 64 + lane];
        const f32x4 x0 = HF == 0 ? acc[kept] : other;
        const f32x4 x1 = HF == 0 ? other : acc[kept];
        acc[lo] = x0 + x1;
        acc[hi] = x0 - x1;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const f32x4 x0 = acc[u], x1 = acc[u + 8];
        acc[u] = x0 + x1;
        acc[u + 8] = x0 - x1;
    }
    const int o0 = 4 * q;
    const bool ok = row_ok && o0 < a.out_o;
    const uint32_t voff = ok ? (uint32_t)((int64_t)row * a.ldy * 2) + (uint32_t)o0 * 2 : kOOB;
    const uint32_t hstride = (uint32_t)a.gsy * 2;
    const f32x4 *bl = beta_l + q * 32;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int h = (u & 3) + 4 * HF + 8 * ((u >> 2) & 1) + 16 * (u >> 3);
        Buf4<uint16_t>::store(acc[u] * bl[h], yr, voff, (uint32_t)h * hstride);
    }
}

// blockDim.x = 128 * Kc (2 <= Kc <= kKparMaxKc), no RoPE.
__global__ __launch_bounds__(kPairThreads * kKparMaxKc, 3) void hadamard_pair_kpar_kernel(HadArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint2 *lut = (uint2 *)smem;
    f32x4 *alpha_l = (f32x4 *)(smem + 256 * 8);   // [Kc][4 q][32 g]
    f32x4 *beta_l = alpha_l + a.Kc * 128;          // [4 q][32 h]
    f32x4 *xch = beta_l + 128;                     // [Kc pairs][2 HF][8][64 lanes]
    const int tid = threadIdx.x, nthr = (int)blockDim.x;
    for (int e = tid; e < 256; e += nthr) {
        float val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) val[j] = (float)((int)(((uint32_t)e >> (6 - 2 * j)) & 3u) - 1);
        lut[e] = uint2{pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3])};
    }
    for (int e = tid; e < a.Kc * 128; e += nthr) {   // e = (c*4 + q)*32 + g
        const int g = e & 31, i0 = 4 * (e >> 5);
        f32x4 va;
#pragma unroll
        for (int j = 0; j < 4; ++j) va[j] = (i0 + j < a.in_o) ? (a.alpha ? a.alpha[g * a.in_o + i0 + j] : 1.f) : 0.f;
        alpha_l[e] = va;
    }
    for (int e = tid; e < 128; e += nthr) {
        const int h = e & 31, o0 = 4 * (e >> 5);
        f32x4 vb;
#pragma unroll
        for (int j = 0; j < 4; ++j) vb[j] = (o0 + j < a.out_o) ? a.beta[h * a.beta_h + o0 + j] * 0.03125f : 0.f;
        beta_l[e] = vb;
    }
    __syncthreads();
    const int wave = tid >> 6, lane = tid & 63;
    const int pair = wave >> 1, hf = wave & 1;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a, 2));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * 2));
    const int n_tiles = (int)ceil_div(a.M, kTile);
    for (int tile = (int)blockIdx.x; tile < n_tiles; tile += (int)gridDim.x) {
        if (hf == 0) kpar_tile<0>(a, tile, pair, lane, lut, alpha_l, beta_l, xch, xr, yr);
        else kpar_tile<1>(a, tile, pair, lane, lut, alpha_l, beta_l, xch, xr, yr);
    }
}

// DENSE: float weights as matrix-core A fragments [32 g][64 lanes] (the
// Hadamard head mixer, one layer), read per tile from memory.
template <bool DENSE>
__global__ __launch_bounds__(kPairThreads, DENSE ? 3 : 4) void hadamard_pair_kernel(HadArgsN an) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint2 *lut = (uint2 *)smem;
    f32x4 *alpha_l = (f32x4 *)(smem + 256 * 8);   // [4 q][32 g]
    f32x4 *beta_l = alpha_l + 128;                 // [4 q][32 h]
    f32x4 *xch = beta_l + 128;                     // [2 HF][8][64 lanes]
    // (layer, first tile) of this workgroup.  Consecutive workgroups go to
    // the 8 XCDs in turn; workgroups 8 (n k + l) + x (l < n) take layer l of
    // tile slot 8 k + x, so the n layers of a tile run on one XCD and read
    // its rows from one L2.  A last partial group of 8 n workgroups keeps
    // slot b / n, layer b % n.
    const int b = (int)blockIdx.x, n = an.n, full = (int)gridDim.x / (8 * n) * (8 * n);
    const int l = b < full ? (b / 8) % n : b % n;
    const int slot = b < full ? (b / (8 * n)) * 8 + b % 8 : b / n;
    const HadArgs &a = an.p[l];
    const int tid = threadIdx.x;
    {
        const int e = tid;   // (q, g) = (e >> 5, e & 31); kPairThreads == 128 entries
        const int g = e & 31, i0 = 4 * (e >> 5);
        // buffer loads (zero past in_o / out_o) with no branch around them,
        // converted after the LUT is built: a conversion or branch right
        // after a load waits for it
        // (no alpha: a resource of no records, every load out of range)
        uint32_t ra[4], rb[4];
        const __amdgpu_buffer_rsrc_t br = make_rsrc(a.beta, (uint32_t)((31 * a.beta_h + a.out_o) * 4));
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(a.alpha, a.alpha ? (uint32_t)(32 * a.in_o * 4) : 0u);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            ra[j] = __builtin_amdgcn_raw_buffer_load_b32(ar, i0 + j < a.in_o ? (uint32_t)(g * a.in_o + i0 + j) * 4 : kOOB,
                                                         0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            rb[j] = __builtin_amdgcn_raw_buffer_load_b32(br, i0 + j < a.out_o ? (uint32_t)(g * a.beta_h + i0 + j) * 4 : kOOB,
                                                         0, 0);
        for (int c = tid; c < 256; c += kPairThreads) {
            float val[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) val[j] = (float)((int)(((uint32_t)c >> (6 - 2 * j)) & 3u) - 1);
            lut[c] = uint2{pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3])};
        }
        f32x4 va, vb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            va[j] = (i0 + j < a.in_o) ? (a.alpha ? __uint_as_float(ra[j]) : 1.f) : 0.f;
            vb[j] = (i0 + j < a.out_o) ? __uint_as_float(rb[j]) * 0.03125f : 0.f;
        }
        alpha_l[e] = va;
        beta_l[e] = vb;
    }
    __syncthreads();
    const int hf = tid >> 6, lane = tid & 63;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a, 2));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * 2));
    const int n_tiles = (int)ceil_div(a.M, kTile);
    const int nb = (int)gridDim.x / an.n;
    for (int tile = slot; tile < n_tiles; tile += nb) {
        if (hf == 0) pair_tile<0, DENSE>(a, tile, lane, lut, alpha_l, beta_l, xch, xr, yr);
        else pair_tile<1, DENSE>(a, tile, lane, lut, alpha_l, beta_l, xch, xr, yr);
    }
}

// ---------------------------------------------------------------- wide layers
// in_o > 16 with several output tiles (n_embd 4096: in_o = out_o = 128).  One
// workgroup of 8 waves takes a (16-token tile, group of 8 output tiles): the
// transformed input of up to S chunks of 16 columns is staged in LDS (wave w
// transforms chunk s0 + w), then wave w contracts output tile nt0 + w over
// the staged chunks, so the input transform is done once per workgroup
// rather than once per output tile, and 8 waves share a token tile.
constexpr int kWideWaves = 8;
constexpr int kWideThreads = 64 * kWideWaves;
template <bool BF16MMA> constexpr int wide_stage() { return BF16MMA ? 8 : 4; }
template <bool BF16MMA> struct XElem;
template <> struct XElem<true> { typedef uint2 type; };
template <> struct XElem<false> { typedef f32x4 type; };

template <bool BF16MMA> constexpr size_t wide_lds_bytes() {
    return (size_t)lut_bytes<BF16MMA>() + (size_t)kWideWaves * 128 * 16 +
           (size_t)wide_stage<BF16MMA>() * 32 * 64 * sizeof(typename XElem<BF16MMA>::type);
}

// alpha[g, i0], alpha[g, i0 + 1] (zeros past in_o); A2: in_o is even.
template <bool A2>
__device__ __forceinline__ f32x2 alpha2(const HadArgs &a, int g, int i0) {
    const float *p = a.alpha + (int64_t)g * a.in_o + i0;
    if (A2) return i0 < a.in_o ? *(const f32x2 *)p : f32x2{0.f, 0.f};
    return f32x2{i0 < a.in_o ? p[0] : 0.f, i0 + 1 < a.in_o ? p[1] : 0.f};
}

template <typename T, bool BF16MMA, bool A4>
__global__ __launch_bounds__(kWideThreads, 1) void hadamard_wide_kernel(HadArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int S = wide_stage<BF16MMA>();
    typedef typename XElem<BF16MMA>::type XE;
    void *lut = smem;
    f32x4 *beta_l = (f32x4 *)(smem + lut_bytes<BF16MMA>());  // [8 local tiles][4][32]
    XE *xs = (XE *)(beta_l + kWideWaves * 128);             // [S][32 g][64 lanes]
    constexpr uint32_t esz = sizeof(T);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t = lane & 15, q = lane >> 4;
    if (tid < 256) {
        const uint32_t byte = (uint32_t)tid;
        float val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) val[j] = (float)((int)((byte >> (6 - 2 * j)) & 3u) - 1);
        if constexpr (BF16MMA) {
            ((uint2 *)lut)[byte] = uint2{pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3])};
        } else {
            ((f32x4 *)lut)[byte] = f32x4{val[0], val[1], val[2], val[3]};
        }
    }
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * esz));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * esz));
    const int n_tiles = (int)ceil_div(a.M, kTile);
    const int ngroups = (int)ceil_div(a.Nt, kWideWaves);
    for (int item = blockIdx.x; item < n_tiles * ngroups; item += gridDim.x) {
        const int tile = item / ngroups, nt0 = (item % ngroups) * kWideWaves, nt = nt0 + wave;
        const int row = tile * kTile + t;
        const bool row_ok = row < a.M;
        const uint32_t xoff = (uint32_t)((int64_t)row * a.ldx * esz);
        const uint32_t yoff = (uint32_t)((int64_t)row * a.ldy * esz);
        __syncthreads();  // LUT ready / previous item done with beta_l and xs
        for (int e = tid; e < kWideWaves * 128; e += kWideThreads) {
            const int lw = e >> 7, h = e & 31, qq = (e >> 5) & 3;
            const int o0 = kNTile * (nt0 + lw) + 4 * qq;
            f32x4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = (o0 + j < a.out_o) ? a.beta[h * a.out_o + o0 + j] * 0.03125f : 0.f;
            beta_l[e] = v;
        }
        f32x4 acc[32];
#pragma unroll
        for (int g = 0; g < 32; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < a.Kc; s0 += S) {
            // transform chunk s0 + wave into LDS slot `wave`
            if (wave < S && s0 + wave < a.Kc) {
                // two passes of 2 columns keep the transform at 64 registers
                // beside the 128 of accumulators
                const int c = s0 + wave;
                const int i0 = kKChunk * c + 4 * q;
                const uint32_t gstride = (uint32_t)a.gsx * esz;
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const int ip = i0 + 2 * p;
                    const uint32_t voff = (row_ok && ip < a.in_o) ? xoff + (uint32_t)ip * esz : kOOB;
                    f32x2 v[32];
#pragma unroll
                    for (int g = 0; g < 32; ++g) {
                        if constexpr (sizeof(T) == 2) {
                            const uint32_t u = __builtin_amdgcn_raw_buffer_load_b32(xr, voff, (uint32_t)g * gstride, 0);
                            v[g] = f32x2{__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u)};
                        } else {
                            v[g] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                                 xr, voff, (uint32_t)g * gstride, 0));
                        }
                    }
#pragma unroll
                    for (int g = 0; g < 32; ++g) {
                        v[g] = v[g] * alpha2<A4>(a, g, ip);
                        if ((g & 7) == 7) __builtin_amdgcn_sched_barrier(0);
                    }
                    fht32<f32x2>(v);
                    XE *dst = xs + (size_t)wave * 32 * 64 + lane;
#pragma unroll
                    for (int g = 0; g < 32; ++g) {
                        if constexpr (BF16MMA)
                            ((uint32_t *)&dst[g * 64])[p] = pack_bf16x2(v[g][0], v[g][1]);
                        else
                            ((f32x2 *)&dst[g * 64])[p] = v[g];
                    }
                }
            }
            __syncthreads();
            if (nt < a.Nt) {
                const int nc = a.Kc - s0 < S ? a.Kc - s0 : S;
                uint4 w0, w1;
                load_w(a, nt, s0, lane, w0, w1);
                for (int j = 0; j < nc; ++j) {
                    uint4 n0 = w0, n1 = w1;
                    if (j + 1 < nc) load_w(a, nt, s0 + j + 1, lane, n0, n1);
                    // staged operands are read group by group next to their products
                    const XE *src = xs + (size_t)j * 32 * 64 + lane;
                    const uint32_t wb[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int g = 0; g < 32; ++g) {
                        const uint32_t byte = (wb[g >> 2] >> (8 * (g & 3))) & 0xffu;
                        const XE xg = src[g * 64];
                        if constexpr (BF16MMA) {
                            const uint2 wa = ((const uint2 *)lut)[byte];
                            acc[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                                __builtin_bit_cast(i16x4, wa), __builtin_bit_cast(i16x4, xg), acc[g], 0, 0, 0);
                        } else {
                            const f32x4 wa = ((const f32x4 *)lut)[byte];
#pragma unroll
                            for (int u = 0; u < 4; ++u)
                                acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[u], xg[u], acc[g], 0, 0, 0);
                        }
                        if ((g & 7) == 7) __builtin_amdgcn_sched_barrier(0);
                    }
                    w0 = n0;
                    w1 = n1;
                }
            }
            __syncthreads();
        }
        if (nt < a.Nt) transform_store<T, true>(a, acc, yr, yoff, row_ok, nt, q, beta_l + (wave - nt) * 128, row);
    }
}

// ---------------------------------------------------------------- wide bf16 layers
// bf16 layers with 16 < in_o <= 128 and out_o <= 128 (n_embd 4096: in_o =
// out_o = 128) on 16x16x32 matrix-core products.  A workgroup of 8 waves
// takes one 16-token tile at a time:
//   1. wave w transforms columns 16w..16w+15 of all 32 groups (alpha, FHT
//      over the groups in registers) and writes them to an LDS stage laid out
//      as the products' B operand: [32-column chunk][group][lane] x 16 bytes,
//      so every later read is one contiguous 1 KB per wave;
//   2. wave w contracts output tile w against the whole stage (32 groups x
//      in_o/32 chunks);
//   3. wave w runs the output transform and beta into an LDS output tile
//      (the stage's space), which leaves as whole contiguous rows (16 bytes
//      per lane, 1 KB per wave and store) instead of 32-byte row pieces.
// The next tile's x is loaded during the last chunk's products and the
// output phase.  Weight codes are stored 4 per byte in base 3 (byte =
// sum_j (code_j + 1) 3^j) and expanded through an 81-entry byte -> 4 x bf16
// table of +-1/32 (the two transforms' 1/sqrt(32)^2, exact in bf16), held in
// 16 copies, entry-major with one 8-byte copy per lane of a 16-lane group.
// (A 9-entry table of bf16 pairs in 64 conflict-free copies was measured
// slower: twice the LDS instructions.)  alpha and beta stay in LDS for the
// whole launch as fp16 (11-bit significand, 2^-12 relative rounding against
// the 2^-9 of the bf16 activations): with the 128 KB stage, float32 copies of
// both would not fit in 160 KB.
constexpr int kW3Copies = 16;
constexpr int kW3Entries = 81;
constexpr int kW3MaxO = 128;  // in_o and out_o limit
constexpr size_t kW3LutBytes = (size_t)kW3Entries * kW3Copies * 8;
constexpr size_t kW3AlphaBytes = (size_t)32 * kW3MaxO * 2;             // [32 g][128 cols] fp16
constexpr size_t kW3BetaBytes = (size_t)32 * kW3MaxO * 2;              // [8 tiles][32 h][16 o] fp16

constexpr int kW3ORow = 32 * kW3MaxO * 2 + 16;                        // output tile row stride (bytes)

static size_t wide3_lds_bytes(int Kc32) {
    const size_t stage = (size_t)Kc32 * 32 * 64 * 16, otile = (size_t)kTile * kW3ORow;
    return kW3LutBytes + kW3AlphaBytes + kW3BetaBytes + (stage > otile ? stage : otile);
}

// Base-3 weight layout [Nt][Kc32][64 lanes][32 groups][2] bytes: lane l of
// (nt, c) holds for group g the bytes of codes
// W[g, 16nt + l%16, 32c + 8(l/16) + 4h .. +3], h = 0, 1 (40 = four zero codes,
// used past out_o / in_o).  Packed code 0b11 is never written by the packer;
// it saturates to +1 here.
__global__ void hadamard_prepare3_kernel(const uint8_t *__restrict__ packed, int in_o, int out_o, int Nt, int Kc32,
                                         uint8_t *__restrict__ kw3) {
    const int64_t total = (int64_t)Nt * Kc32 * 64 * 64;
    const int kp4 = (int)ceil_div(in_o, 4);
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int h = (int)(e & 1);
        const int g = (int)((e >> 1) & 31);
        const int lane = (int)((e >> 6) & 63);
        const int64_t tc = e >> 12;
        const int c = (int)(tc % Kc32);
        const int nt = (int)(tc / Kc32);
        const int o = kNTile * nt + (lane & 15);
        const int i0 = 32 * c + 8 * (lane >> 4) + 4 * h;
        int b = 40;
        if (o < out_o && i0 < in_o) {
            const uint32_t p = packed[((int64_t)g * out_o + o) * kp4 + i0 / 4];
            b = 0;
            int w3 = 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = (int)((p >> (6 - 2 * j)) & 3u);
                b += (d > 2 ? 2 : d) * w3;
                w3 *= 3;
            }
        }
        kw3[e] = (uint8_t)b;
    }
}

// Groups G0..G1-1 of the lane's 4 transform columns as raw bf16.
template <int G0 = 0, int G1 = 32>
__device__ __forceinline__ void wide3_load_x(__amdgpu_buffer_rsrc_t xr, uint32_t voff, uint32_t gstride,
                                             u32x2 (&r)[32]) {
#pragma unroll
    for (int g = G0; g < G1; ++g) r[g] = __builtin_amdgcn_raw_buffer_load_b64(xr, voff, (uint32_t)g * gstride, 0);
}

// The lane's 4 columns of one row, scaled by alpha (fp16 in LDS, al[g * 128])
// and transformed over the 32 groups, into the stage as bf16 (xdst[g * 128]
// in uint2 units).  Two passes of 2 columns keep the transform at 64
// registers.
__device__ __forceinline__ void wide3_transform_x(const u32x2 (&xraw)[32], const _Float16 *al, uint2 *xdst) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        f32x2 v[32];
#pragma unroll
        for (int g = 0; g < 32; ++g) {
            const uint32_t u = p ? xraw[g].y : xraw[g].x;
            const _Float16 *ag = al + g * kW3MaxO + 2 * p;
            v[g] = f32x2{__uint_as_float(u << 16) * (float)ag[0], __uint_as_float(u & 0xffff0000u) * (float)ag[1]};
        }
        fht32<f32x2>(v);
#pragma unroll
        for (int g = 0; g < 32; ++g) ((uint32_t *)&xdst[g * 128])[p] = pack_bf16x2(v[g][0], v[g][1]);
    }
}

// GS: 128 for in_o = out_o = 128 with unpadded groups (the n_embd 4096
// layers: strides fixed at compile time), 0 for any other shape.
// DENSE: dense bf16 weights (the head mixer at head_dim 128) as 16x16x32
// A fragments [Nt][Kc32][32 g][64 lanes] x 16 bytes, streamed from global
// memory a few groups ahead of their products, instead of the code table.
template <int GS, bool DENSE = false>
__global__ __launch_bounds__(kWideThreads, 1) void hadamard_wide3_kernel(HadArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint2 *lut = (uint2 *)smem;                                          // [81 entries][16 copies]
    _Float16 *alpha_l = (_Float16 *)(smem + kW3LutBytes);                // [32 g][128 cols]
    _Float16 *beta_l = (_Float16 *)(smem + kW3LutBytes + kW3AlphaBytes); // [8 tiles][32 h][16 o]
    uint4 *xs = (uint4 *)(smem + kW3LutBytes + kW3AlphaBytes + kW3BetaBytes);  // [Kc32][32 g][64 lanes]
    unsigned char *ostage = (unsigned char *)xs;  // after the products: the output tile
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t = lane & 15, q = lane >> 4;
    for (int e = tid; e < (DENSE ? 0 : kW3Entries * kW3Copies); e += kWideThreads) {
        int r = e / kW3Copies;
        float val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            val[j] = (float)(r % 3 - 1) * 0.03125f;
            r /= 3;
        }
        lut[e] = uint2{pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3])};
    }
    for (int e = tid; e < 32 * kW3MaxO; e += kWideThreads) {
        const int g = e / kW3MaxO, i = e % kW3MaxO;
        // the two transforms' 1/32 rides on the code table; dense weights
        // carry no such factor, so it goes on alpha (exact: a power of two)
        const float a32 = DENSE ? 0.03125f : 1.f;
        alpha_l[e] = (_Float16)(i < a.in_o ? (a.alpha ? a.alpha[g * a.in_o + i] : 1.f) * a32 : 0.f);
        const int o = kNTile * (e >> 9) + (e & 15), h = (e >> 4) & 31;  // e = (nt*32 + h)*16 + o%16
        beta_l[e] = (_Float16)(o < a.out_o ? a.beta[h * a.beta_h + o] : 0.f);
    }
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a, 2));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * 2));
    const int n_tiles = (int)ceil_div(a.M, kTile);
    const int Kc32 = (a.in_o + 31) >> 5;
    const uint2 *lut_l = lut + (lane & 15);
    const uint32_t gstride = (uint32_t)(GS ? GS : a.gsx) * 2;
    // this wave's transform columns and their place in the stage
    const int i0 = 16 * wave + 4 * q;
    uint2 *xdst = (uint2 *)(xs + (size_t)(i0 >> 5) * 32 * 64 + t + 16 * ((i0 >> 3) & 3)) + ((i0 >> 2) & 1);
    const bool xwave = wave < 2 * Kc32;
    // every wave runs the products (uniform control flow keeps the
    // accumulators in registers across the barriers); a wave past the last
    // output tile reads tile 0's weights and its results are never stored
    const int wt = wave < a.Nt ? wave : 0;
    const uint4 *wsrc = DENSE ? nullptr : (const uint4 *)(a.kw3 + ((int64_t)wt * Kc32 * 64 + lane) * 64);
    const uint4 *wdn = DENSE ? (const uint4 *)a.kw + (int64_t)wt * Kc32 * 32 * 64 + lane : nullptr;  // + (c*32+g)*64
    constexpr int RD = 4;  // DENSE: fragments in flight ahead of their products
    uint4 ring[RD];
    const _Float16 *bl = beta_l + wave * 512 + 4 * q;
    const _Float16 *al = alpha_l + i0;
    auto x_off = [&](int tile) -> uint32_t {
        const int row = tile * kTile + t;
        return (row < a.M && i0 < a.in_o) ? x_row_off(a, row, 2) + (uint32_t)i0 * 2 : kOOB;
    };
    // x of the first tile; later tiles are loaded during the contraction of
    // the one before, so their load latency overlaps the matrix work
    u32x2 xraw[32];
    if (xwave && (int)blockIdx.x < n_tiles) wide3_load_x(xr, x_off(blockIdx.x), gstride, xraw);
    for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const int next = tile + gridDim.x;
        lds_barrier();  // tables ready / previous tile done with the stage
        if (xwave) wide3_transform_x(xraw, al, xdst);
        if (DENSE) {
            // the first fragments load while the other waves finish their
            // transforms
#pragma unroll
            for (int j = 0; j < RD; ++j) ring[j] = wdn[j * 64];
        }
        lds_barrier();
        f32x4 acc[32];
        const bool pf = xwave && next < n_tiles;
        const uint32_t pf_off = pf ? x_off(next) : kOOB;
#pragma unroll
        for (int g = 0; g < 32; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (DENSE) {
            for (int c = 0; c < Kc32; ++c) {
                const uint4 *xsrc = xs + (size_t)c * 32 * 64 + lane;
                const bool more = c + 1 < Kc32;
#pragma unroll
                for (int g = 0; g < 32; ++g) {
                    const uint4 wa = ring[g % RD];
                    if (g == 32 - RD && !more) {
                        // the tile's last weight load is issued: the next
                        // tile's x (groups 0-15) follows without holding
                        // up any weight wait
                        __builtin_amdgcn_sched_barrier(0);
                        if (pf) wide3_load_x<0, 16>(xr, pf_off, gstride, xraw);
                    }
                    if (g < 32 - RD) ring[g % RD] = wdn[(c * 32 + g + RD) * 64];
                    else if (more) ring[g % RD] = wdn[((c + 1) * 32 + g - (32 - RD)) * 64];
                    const uint4 xb = xsrc[g * 64];
                    acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wa),
                                                                     __builtin_bit_cast(bf16x8, xb), acc[g], 0, 0, 0);
                }
            }
        } else {
            // one 32-column chunk: 32 products
            auto chunk = [&](int c, const uint4 (&w)[4]) {
                const uint4 *xsrc = xs + (size_t)c * 32 * 64 + lane;
#pragma unroll
                for (int g = 0; g < 32; ++g) {
                    const uint32_t word = w[g >> 3][(g >> 1) & 3] >> (16 * (g & 1));
                    const uint2 lo = lut_l[(word & 0xffu) * kW3Copies];
                    const uint2 hi = lut_l[((word >> 8) & 0xffu) * kW3Copies];
                    const uint4 xb = xsrc[g * 64];
                    acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, uint4{lo.x, lo.y, hi.x, hi.y}), __builtin_bit_cast(bf16x8, xb),
                        acc[g], 0, 0, 0);
                }
            };
            uint4 w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = wsrc[j];
            for (int c = 0; c + 1 < Kc32; ++c) {
                uint4 wn[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) wn[j] = wsrc[(c + 1) * 256 + j];
                chunk(c, w);
#pragma unroll
                for (int j = 0; j < 4; ++j) w[j] = wn[j];
            }
            // the next tile's x: groups 0-15 behind the last chunk (whose
            // weights are already in registers, so no weight load waits
            // behind them), groups 16-31 once the output tile is written and
            // the accumulators are free
            __builtin_amdgcn_sched_barrier(0);
            if (pf) wide3_load_x<0, 16>(xr, pf_off, gstride, xraw);
            chunk(Kc32 - 1, w);
        }
        lds_barrier();  // every wave is done with the stage: it now takes the output tile
        {
            // output transform over h and beta, into the LDS output tile
            // [16 rows][32 h][128 o] (rows padded by 16 bytes: the 16 rows
            // of a write fall on different banks)
            fht32x4(acc);
            unsigned char *od = ostage + t * kW3ORow + (kNTile * wave + 4 * q) * 2;
            const int orow = tile * kTile + t, o0 = kNTile * wave + 4 * q;
            // rotary embedding: the same two (cos, sin) pairs for all 32 groups
            const bool rope = a.rope != nullptr;
            const f32x4 cs = (rope && orow < a.M && o0 < a.out_o) ? rope_cs(a, orow, o0) : f32x4{1.f, 0.f, 1.f, 0.f};
#pragma unroll
            for (int h0 = 0; h0 < 32; h0 += 8) {
                uint2 b8[8];  // beta of 8 output groups, read together
#pragma unroll
                for (int j = 0; j < 8; ++j) b8[j] = *(const uint2 *)(bl + (h0 + j) * 16);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const _Float16 *b = (const _Float16 *)&b8[j];
                    f32x4 r = acc[h0 + j] * f32x4{(float)b[0], (float)b[1], (float)b[2], (float)b[3]};
                    if (rope) r = rope_apply(r, cs);
                    *(uint2 *)(od + (h0 + j) * kW3MaxO * 2) = uint2{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (pf) wide3_load_x<16, 32>(xr, pf_off, gstride, xraw);
        }
        lds_barrier();
        // the whole tile leaves as contiguous rows: each lane takes 8 outputs
        // (16 bytes) of a row, 1 KB per wave and instruction
#pragma unroll 4
        for (int r = 0; r < kTile; ++r) {
            const int orow = tile * kTile + r;
            const uint4 v = *(const uint4 *)(ostage + r * kW3ORow + tid * 16);
            if (GS == kW3MaxO) {
                const uint32_t voff = orow < a.M ? (uint32_t)((int64_t)orow * a.ldy * 2) + (uint32_t)tid * 16 : kOOB;
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), yr, voff, 0, 0);
            } else {
                // group stride gsy: two 4-output stores at h*gsy + o
                const int h = tid >> 4, o = (tid & 15) * 8;
                const uint32_t base = (uint32_t)((int64_t)orow * a.ldy * 2) + (uint32_t)(h * a.gsy + o) * 2;
                const uint32_t v0 = (orow < a.M && o < a.out_o) ? base : kOOB;
                const uint32_t v1 = (orow < a.M && o + 4 < a.out_o) ? base + 8 : kOOB;
                __builtin_amdgcn_raw_buffer_store_b64(u32x2{v.x, v.y}, yr, v0, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b64(u32x2{v.z, v.w}, yr, v1, 0, 0);
            }
        }
    }
}

// ---------------------------------------------------------------- decode-sized batches
// With a few 16-token tiles the wide3 kernel runs one workgroup per tile, so
// a whole layer's codes stream through a handful of CUs and the launch lasts
// as long as one workgroup's chunk loop.  Here a workgroup takes one (token
// tile, output tile, layer): its 8 waves stage the tile's transformed input
// as the wide3 kernel does, wave w contracts groups 4w..4w+3 over every
// chunk, the 32 group products meet in LDS and 4 waves run the output
// transform, one column quad each.  Every rounding and every sum follows
// the wide3 kernel's order, so both give bitwise the same rows; the input
// transform is repeated per output tile, which a few rows make cheap.
#ifndef WALSH_SPLIT_ROWS
#define WALSH_SPLIT_ROWS 256
#endif
constexpr int kSplitRows = WALSH_SPLIT_ROWS;            // row counts up to this take the split kernel
constexpr size_t kSplitBetaBytes = (size_t)32 * kNTile * 2;  // [32 h][16 o] fp16

static size_t split3_lds_bytes(int Kc32) {
    const size_t stage = (size_t)Kc32 * 32 * 64 * 16, part = (size_t)32 * 64 * 16;
    return kW3LutBytes + kW3AlphaBytes + kSplitBetaBytes + (stage > part ? stage : part);
}

// Grid: x = token tile * Nt + output tile, y = layer of `an`.  GS and DENSE
// as for the wide3 kernel.
template <int GS, bool DENSE>
__global__ __launch_bounds__(kWideThreads, 1) void hadamard_split3_kernel(HadArgsN an) {
    extern __shared__ __align__(16) unsigned char smem[];
    const HadArgs a = load_args(an.p[blockIdx.y]);
    uint2 *lut = (uint2 *)smem;                                           // [81 entries][16 copies]
    _Float16 *alpha_l = (_Float16 *)(smem + kW3LutBytes);                 // [32 g][128 cols]
    _Float16 *beta_l = (_Float16 *)(smem + kW3LutBytes + kW3AlphaBytes);  // [32 h][16 o] of this tile
    uint4 *xs = (uint4 *)(smem + kW3LutBytes + kW3AlphaBytes + kSplitBetaBytes);  // [Kc32][32 g][64 lanes]
    f32x4 *part = (f32x4 *)xs;  // after the products: [32 g][64 lanes]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t = lane & 15, q = lane >> 4;
    const int nt = (int)blockIdx.x % a.Nt, tile = (int)blockIdx.x / a.Nt;
    const int Kc32 = (a.in_o + 31) >> 5;

    // every load first, so one memory round trip covers them all, in the
    // order of use (vector loads complete in order): the tile's input, alpha
    // and this output tile's beta, this wave's weights of groups 4w..4w+3
    // for every chunk, the output waves' rotary coefficients
    const int i0 = 16 * wave + 4 * q;
    const bool xwave = wave < 2 * Kc32;
    // Few valid rows in the tile (decode): a thread transforms one column
    // pair of one valid row (unit tid: row tid / (in_o / 2), pair tid % (in_o
    // / 2)) instead of 4 columns of each of the 16 row slots, most of them
    // rows past M.  The stage slots of rows past M are then left unwritten:
    // a product column is one row, and those rows are not stored.
    const int mt = min(kTile, a.M - tile * kTile), hp = a.in_o >> 1;
    const bool narrow = (a.in_o & 31) == 0 && mt * hp <= kWideThreads;   // workgroup-uniform
    const int n_tok = tid / hp, n_col = 2 * (tid - n_tok * hp);
    const bool n_ok = narrow && n_tok < mt;
    // Full tiles of contiguous 4096-element rows: the tile (16 rows x 8 KB)
    // comes straight into the stage region with buffer-to-LDS loads, a whole
    // 1 KB row segment per instruction (the per-thread loads below touch 16
    // rows per instruction, 32 bytes of each, and queue up behind each
    // other); 16-byte chunk p of row t sits at position p ^ t of its 256-byte
    // window, so that one column's 16 rows fall on distinct banks when each
    // thread reads its 32 groups back.
    const bool lds_x = !narrow && a.in_o == 128 && a.gsx == 128;   // workgroup-uniform
    u32x2 xraw[32];
    uint32_t xn[32];
    {
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a, 2));
        const uint32_t gstride = (uint32_t)(GS ? GS : a.gsx) * 2;
        if (narrow) {
            const uint32_t voff = n_ok ? x_row_off(a, tile * kTile + n_tok, 2) + (uint32_t)n_col * 2 : kOOB;
#pragma unroll
            for (int g = 0; g < 32; ++g) xn[g] = __builtin_amdgcn_raw_buffer_load_b32(xr, voff, (uint32_t)g * gstride, 0);
        } else if (lds_x) {
            const int w = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int seg = w * 16 + i, tr = seg >> 3, sg = seg & 7;   // row of the tile, 1 KB segment
                const int row = tile * kTile + tr;
                const uint32_t off =
                    row < a.M ? x_row_off(a, row, 2) + (uint32_t)(sg * 1024 + ((lane ^ tr) << 4)) : kOOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    xr, (__attribute__((address_space(3))) void *)((unsigned char *)xs + tr * 8192 + sg * 1024), 16,
                    off, 0, 0, 0);
            }
        } else if (xwave) {
            const int row = tile * kTile + t;
            const uint32_t voff = (row < a.M && i0 < a.in_o) ? x_row_off(a, row, 2) + (uint32_t)i0 * 2 : kOOB;
            wide3_load_x(xr, voff, gstride, xraw);
        }
    }
    // (buffer loads, zero past their ranges, and no arithmetic on the loaded
    // values until they are used: a conversion right after a load would wait
    // for every load before it)
    const float a32 = DENSE ? 0.03125f : 1.f;  // the dense weights' share of the transforms' 1/32
    constexpr int kAv = 32 * kW3MaxO / kWideThreads;
    uint32_t avr[kAv];
    {
        // (no alpha: a resource of no records, every load out of range)
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(a.alpha, a.alpha ? (uint32_t)(32 * a.in_o * 4) : 0u);
#pragma unroll
        for (int k = 0; k < kAv; ++k) {
            const int e = tid + k * kWideThreads, g = e / kW3MaxO, i = e % kW3MaxO;
            avr[k] = __builtin_amdgcn_raw_buffer_load_b32(ar, i < a.in_o ? (uint32_t)(g * a.in_o + i) * 4 : kOOB, 0, 0);
        }
    }
    const int bo = kNTile * nt + (tid & 15);
    const __amdgpu_buffer_rsrc_t br = make_rsrc(a.beta, (uint32_t)((31 * a.beta_h + a.out_o) * 4));
    const uint32_t bvr = __builtin_amdgcn_raw_buffer_load_b32(
        br, bo < a.out_o ? (uint32_t)((tid >> 4) * a.beta_h + bo) * 4 : kOOB, 0, 0);
    uint2 wv[4];
    uint4 wd[4][4];
    {
        const __amdgpu_buffer_rsrc_t kr =
            DENSE ? make_rsrc(a.kw, (uint32_t)(a.Nt * Kc32 * 32768)) : make_rsrc(a.kw3, (uint32_t)(a.Nt * Kc32 * 4096));
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (c < Kc32) {
                if constexpr (DENSE) {
                    const uint32_t off = (uint32_t)((((nt * Kc32 + c) * 32 + 4 * wave) * 64 + lane) * 16);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        wd[c][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, j * 1024, 0));
                } else {
                    wv[c] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                          kr, (uint32_t)(((nt * Kc32 + c) * 64 + lane) * 64 + 8 * wave), 0, 0));
                }
            }
        }
    }
    // the output waves' rotary (cos, sin): wave w < 4 takes outputs
    // 4w..4w+3 of the tile, lane = (token tt, output jj)
    // (waves w and w + 4 both take outputs 4 (w % 4) .. + 3, groups h of
    // their half: [16 (w / 4), 16 (w / 4) + 16))
    const int ow = wave & 3, h0 = 16 * (wave >> 2);
    const int tt = lane >> 2, jj = lane & 3, o16 = 4 * ow + jj;
    const int orow = tile * kTile + tt, o = kNTile * nt + o16;
    const bool ok = orow < a.M && o < a.out_o;
    const bool rope = a.rope != nullptr;
    const bool cs_ok = rope && ok;
    u32x2 csr = {0u, 0u};
    if (rope) {
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.rope, (uint32_t)(a.rope_T * a.rope_D * 4));
        const uint32_t off = cs_ok ? (uint32_t)((((orow + a.rope_row0) % a.rope_T) * (a.rope_D >> 1) + ((o % a.rope_D) >> 1)) * 8)
                                   : kOOB;
        csr = __builtin_amdgcn_raw_buffer_load_b64(rr, off, 0, 0);
    }

    for (int e = tid; e < (DENSE ? 0 : kW3Entries * kW3Copies); e += kWideThreads) {
        int r = e / kW3Copies;
        float val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            val[j] = (float)(r % 3 - 1) * 0.03125f;
            r /= 3;
        }
        lut[e] = uint2{pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3])};
    }
#pragma unroll
    for (int k = 0; k < kAv; ++k) {
        const int i = (tid + k * kWideThreads) % kW3MaxO;
        alpha_l[tid + k * kWideThreads] = (_Float16)(i < a.in_o ? (a.alpha ? __uint_as_float(avr[k]) : 1.f) * a32 : 0.f);
    }
    beta_l[tid] = (_Float16)(bo < a.out_o ? __uint_as_float(bvr) : 0.f);
    if (lds_x) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's share of the tile is in LDS
    lds_barrier();  // tables ready
    if (lds_x) {
        // the thread's 4 columns i0..i0+3 of row t in every group: byte
        // g * 256 + 2 i0 of the row, chunk p = 16 g + i0 / 8 at p ^ t
        const unsigned char *xrow = (const unsigned char *)xs + t * 8192;
#pragma unroll
        for (int g = 0; g < 32; ++g) {
            const int p = 16 * g + (i0 >> 3);
            xraw[g] = *(const u32x2 *)(xrow + (p >> 6) * 1024 + (((p & 63) ^ t) << 4) + (i0 & 7) * 2);
        }
        lds_barrier();  // every thread holds its columns: the stage region is free
    }
    if (narrow) {
        // the column pair as one pass of wide3_transform_x: the same
        // products, transform and roundings
        if (n_ok) {
            f32x2 v[32];
#pragma unroll
            for (int g = 0; g < 32; ++g) {
                const uint32_t u = xn[g];
                const _Float16 *ag = alpha_l + g * kW3MaxO + n_col;
                v[g] = f32x2{__uint_as_float(u << 16) * (float)ag[0], __uint_as_float(u & 0xffff0000u) * (float)ag[1]};
            }
            fht32<f32x2>(v);
            // stage position of (row n_tok, column n_col): chunk n_col / 32,
            // lane n_tok + 16 ((n_col / 8) % 4), bf16 element n_col % 8
            uint32_t *dst = (uint32_t *)(xs + (size_t)(n_col >> 5) * 32 * 64 + n_tok + 16 * ((n_col >> 3) & 3)) +
                            ((n_col & 7) >> 1);
#pragma unroll
            for (int g = 0; g < 32; ++g) dst[g * 64 * 4] = pack_bf16x2(v[g][0], v[g][1]);
        }
    } else if (xwave || lds_x) {
        wide3_transform_x(xraw, alpha_l + i0,
                          (uint2 *)(xs + (size_t)(i0 >> 5) * 32 * 64 + t + 16 * ((i0 >> 3) & 3)) + ((i0 >> 2) & 1));
    }
    lds_barrier();  // stage ready

    f32x4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint4 *xsrc = xs + 4 * wave * 64 + lane;
    const uint2 *lut_l = lut + (lane & 15);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (c < Kc32) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint4 wa;
                if constexpr (DENSE) {
                    wa = wd[c][j];
                } else {
                    const uint32_t word = (j < 2 ? wv[c].x : wv[c].y) >> (16 * (j & 1));
                    const uint2 lo = lut_l[(word & 0xffu) * kW3Copies];
                    const uint2 hi = lut_l[((word >> 8) & 0xffu) * kW3Copies];
                    wa = uint4{lo.x, lo.y, hi.x, hi.y};
                }
                const uint4 xb = xsrc[(c * 32 + j) * 64];
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wa),
                                                                 __builtin_bit_cast(bf16x8, xb), acc[j], 0, 0, 0);
            }
        }
    }
    lds_barrier();  // every wave is done with the stage: it now takes the products
#pragma unroll
    for (int j = 0; j < 4; ++j) part[(4 * wave + j) * 64 + lane] = acc[j];
    lds_barrier();
    // waves w and w + 4: outputs 4 (w % 4)..+3 of the tile, lane = (token tt,
    // output jj), so one read instruction covers 64 consecutive floats; both
    // run the output transform, each stores half of the 32 groups (two
    // shorter store chains per SIMD instead of one)
    const float *pp = (const float *)part + (tt + 16 * ow) * 4 + jj;
    float v[32];
#pragma unroll
    for (int g = 0; g < 32; ++g) v[g] = pp[g * 256];
    fht32<float>(v);
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * 2));
    const uint32_t voff = ok ? (uint32_t)((int64_t)orow * a.ldy * 2) + (uint32_t)o * 2 : kOOB;
    const uint32_t hstride = (uint32_t)(GS ? GS : a.gsy) * 2;
    const f32x2 cs = cs_ok ? f32x2{__uint_as_float(csr.x), __uint_as_float(csr.y)} : f32x2{1.f, 0.f};
#pragma unroll
    for (int hi = 0; hi < 16; ++hi) {
        const int h = h0 + hi;
        float r = (h0 ? v[16 + hi] : v[hi]) * (float)beta_l[h * kNTile + o16];
        if (rope) {
            // the other element of the pair (lane ^ 1, a DPP quad permutation)
            const float p = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(r), 0xB1, 0xF, 0xF, true));
            r = (jj & 1) ? rope_odd(p, r, cs[0], cs[1]) : rope_even(r, p, cs[0], cs[1]);
        }
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(r), yr, voff, (uint32_t)h * hstride, 0);
    }
}

// Launches the split kernel over `an` (n layers of M rows each, shapes the
// wide3 kernel takes).
static void split3_launch(const HadArgsN &an, bool gs128, bool dense, hipStream_t s) {
    const HadArgs &a = an.p[0];
    const size_t lds = split3_lds_bytes((a.in_o + 31) / 32);
    const dim3 G((unsigned)(ceil_div(a.M, kTile) * a.Nt), (unsigned)an.n), B(kWideThreads);
    if (dense) launch(hadamard_split3_kernel<0, true>, G, B, lds, s, an);
    else if (gs128) launch(hadamard_split3_kernel<128, false>, G, B, lds, s, an);
    else launch(hadamard_split3_kernel<0, false>, G, B, lds, s, an);
}

// ---------------------------------------------------------------- fused SwiGLU
// h = silu(gate(x)) * up(x) for two Hadamard linears sharing the input x
// (SwiGLUMLP.forward, src/model/chassis.py:498-504, whose gate_proj/up_proj
// are HadamardTernaryLinearTuple layers).  A work item is one 16-token tile
// and one 16-wide output tile: the gate result (after its output transform
// and beta) waits in an LDS stash while the up projection runs, then
// silu(g)*u is written once.  `g` and `u` carry the per-projection weights,
// alpha and beta; x/y geometry is read from `g`.
template <bool BF16MMA> struct Stash;
template <> struct Stash<true> { typedef uint2 type; };   // 4 x bf16
template <> struct Stash<false> { typedef f32x4 type; };  // 4 x f32

__device__ __forceinline__ float silu_fast(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
}

template <typename T, bool BF16MMA, bool VEC, bool KC1>
__global__ __launch_bounds__(kThreads, (BF16MMA && KC1) ? 2 : 1) void hadamard_swiglu_kernel(HadArgs g, HadArgs u) {
    extern __shared__ __align__(16) unsigned char smem[];
    typedef typename Stash<BF16MMA>::type SType;
    void *lut = smem;
    f32x4 *ag_l = (f32x4 *)(smem + lut_bytes<BF16MMA>());
    f32x4 *au_l = ag_l + g.Kc * 128;
    f32x4 *bg_l = au_l + g.Kc * 128;
    f32x4 *bu_l = bg_l + g.Nt * 128;
    SType *stash = (SType *)(bu_l + g.Nt * 128);     // [kWaves][32][64]

    const int tid = threadIdx.x;
    {
        const uint32_t byte = (uint32_t)tid;
        float val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) val[j] = (float)((int)((byte >> (6 - 2 * j)) & 3u) - 1);
        if constexpr (BF16MMA) {
            uint2 e;
            e.x = pack_bf16x2(val[0], val[1]);
            e.y = pack_bf16x2(val[2], val[3]);
            ((uint2 *)lut)[byte] = e;
        } else {
            ((f32x4 *)lut)[byte] = f32x4{val[0], val[1], val[2], val[3]};
        }
    }
    for (int e = tid; e < g.Kc * 128; e += kThreads) {
        const int gg = e & 31, i0 = 4 * (e >> 5);
        f32x4 va, vb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool ok = i0 + j < g.in_o;
            va[j] = ok ? g.alpha[gg * g.in_o + i0 + j] : 0.f;
            vb[j] = ok ? u.alpha[gg * g.in_o + i0 + j] : 0.f;
        }
        ag_l[e] = va;
        au_l[e] = vb;
    }
    for (int e = tid; e < g.Nt * 128; e += kThreads) {
        const int h = e & 31, o0 = 4 * (e >> 5);
        f32x4 va, vb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool ok = o0 + j < g.out_o;
            va[j] = ok ? g.beta[h * g.out_o + o0 + j] * 0.03125f : 0.f;
            vb[j] = ok ? u.beta[h * g.out_o + o0 + j] * 0.03125f : 0.f;
        }
        bg_l[e] = va;
        bu_l[e] = vb;
    }
    __syncthreads();

    constexpr uint32_t esz = sizeof(T);
    // with fewer working waves than wavefronts, the idle one rotates with
    // the workgroup index, so the working waves of the workgroups on a CU
    // spread over all four SIMDs instead of the same three
    const int lane = tid & 63;
    const int wave = ((tid >> 6) - (int)blockIdx.x) & (kWaves - 1);
    const int t = lane & 15, q = lane >> 4;
    SType *st = stash + wave * 32 * 64;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.x, (uint32_t)((int64_t)g.M * g.ldx * esz));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(g.y, (uint32_t)((int64_t)g.M * g.ldy * esz));
    const int n_items = (int)ceil_div(g.M, kTile) * g.Nt;
    const int wt = g.wave_tiles > 0 ? g.wave_tiles : kWaves;
    if (wave >= wt) return;   // after the set-up barrier; the item loop has none
    const int stride = gridDim.x * wt;

    for (int item = blockIdx.x * wt + wave; item < n_items; item += stride) {
        const int tile = item / g.Nt, nt = item - tile * g.Nt;
        const int row = tile * kTile + t;
        const bool row_ok = row < g.M;
        const uint32_t xoff = (uint32_t)((int64_t)row * g.ldx * esz);
        const uint32_t yoff = (uint32_t)((int64_t)row * g.ldy * esz);
        f32x4 acc[32];
        // gate (single input chunk: transform before the accumulators are live)
        if constexpr (KC1) {
            XM<BF16MMA> xm;
            load_transform<T, BF16MMA, VEC>(g, xr, xoff, row_ok, 0, q, ag_l, xm);
#pragma unroll
            for (int k = 0; k < 32; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
            contract<BF16MMA>(g, nt, 0, lane, xm, lut, acc);
        } else {
#pragma unroll
            for (int k = 0; k < 32; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
            for (int c = 0; c < g.Kc; ++c) {
                XM<BF16MMA> xm;
                load_transform<T, BF16MMA, VEC>(g, xr, xoff, row_ok, c, q, ag_l, xm);
                contract<BF16MMA>(g, nt, c, lane, xm, lut, acc);
            }
        }
        fht32x4(acc);
        {
            // beta from LDS four groups at a time, so the reads of a batch
            // overlap (one at a time, each waited for, they serialise)
            const f32x4 *bl = bg_l + (nt * 4 + q) * 32;
#pragma unroll
            for (int h0 = 0; h0 < 32; h0 += 4) {
                f32x4 b4[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) b4[j] = bl[h0 + j];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int h = h0 + j;
                    const f32x4 v = acc[h] * b4[j];
                    if constexpr (BF16MMA) {
                        uint2 e;
                        e.x = pack_bf16x2(v.x, v.y);
                        e.y = pack_bf16x2(v.z, v.w);
                        st[h * 64 + lane] = e;
                    } else {
                        st[h * 64 + lane] = v;
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // up
        if constexpr (KC1) {
            XM<BF16MMA> xm;
            load_transform<T, BF16MMA, VEC>(g, xr, xoff, row_ok, 0, q, au_l, xm);
#pragma unroll
            for (int k = 0; k < 32; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
            contract<BF16MMA>(u, nt, 0, lane, xm, lut, acc);
        } else {
#pragma unroll
            for (int k = 0; k < 32; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
            for (int c = 0; c < g.Kc; ++c) {
                XM<BF16MMA> xm;
                load_transform<T, BF16MMA, VEC>(g, xr, xoff, row_ok, c, q, au_l, xm);
                contract<BF16MMA>(u, nt, c, lane, xm, lut, acc);
            }
        }
        fht32x4(acc);
        const int o0 = kNTile * nt + 4 * q;
        const uint32_t hstride = (uint32_t)g.gsy * esz;
        const f32x4 *bl = bu_l + (nt * 4 + q) * 32;
        uint32_t voff[4];
        if (VEC) {
            voff[0] = (row_ok && o0 < g.out_o) ? yoff + (uint32_t)o0 * esz : kOOB;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) voff[j] = (row_ok && o0 + j < g.out_o) ? yoff + (uint32_t)(o0 + j) * esz : kOOB;
        }
        // beta and the stashed gate four groups at a time (reads of a batch
        // in flight together)
#pragma unroll
        for (int h0 = 0; h0 < 32; h0 += 4) {
            f32x4 b4[4];
            SType e4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                b4[j] = bl[h0 + j];
                e4[j] = st[(h0 + j) * 64 + lane];
            }
#pragma unroll
            for (int j4 = 0; j4 < 4; ++j4) {
                const int h = h0 + j4;
                const f32x4 uv = acc[h] * b4[j4];
                f32x4 gv;
                if constexpr (BF16MMA) {
                    const uint2 e = e4[j4];
                    gv.x = __uint_as_float(e.x << 16);
                    gv.y = __uint_as_float(e.x & 0xffff0000u);
                    gv.z = __uint_as_float(e.y << 16);
                    gv.w = __uint_as_float(e.y & 0xffff0000u);
                } else {
                    gv = e4[j4];
                }
                f32x4 hv;
#pragma unroll
                for (int j = 0; j < 4; ++j) hv[j] = silu_fast(gv[j]) * uv[j];
                if (VEC) {
                    Buf4<T>::store(hv, yr, voff[0], (uint32_t)h * hstride);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) Buf4<T>::store1(hv[j], yr, voff[j], (uint32_t)h * hstride);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// ---------------------------------------------------------------- fused MLP
// down(silu(gate(x)) * up(x)) (SwiGLUMLP.forward, chassis.py:498-504) in one
// launch, for bf16 rows with in_o <= 16 (n_embd 512), a hidden width of two
// or three 16-wide tiles (16 < hid_o <= 48) and a down projection with
// out_o <= 16.  A workgroup takes one 16-token tile at a time:
//   - wave nt < Nt runs the SwiGLU item of hidden tile nt as
//     hadamard_swiglu_kernel does (gate into its LDS area, up, silu(g) u),
//     rounds the hidden values to bf16 as that kernel's store does, and runs
//     the down projection's input transform of chunk nt on them in
//     registers: hidden tile nt's columns 16 nt + 4q .. +3 are exactly
//     chunk nt's in the lane layout load_transform reads, so nothing is
//     rearranged.  The transformed chunk (bf16, 16 KB) replaces the gate
//     stash in the wave's area;
//   - after a barrier wave 3 contracts the chunks in order into one
//     accumulator chain (the one-wavefront chunk loop's order) and, after a
//     second barrier that frees the areas for the next tile, runs the output
//     transform, beta and the stores, overlapping the next tile's items.
// The hidden activation never leaves the CU, and the output equals
// walsh_hadamard_swiglu_fwd followed by the down projection bitwise.
constexpr int kMlpDownWave = 3;

__global__ __launch_bounds__(kThreads, 2) void hadamard_mlp_kernel(HadArgs g, HadArgs u, HadArgs d) {
    extern __shared__ __align__(16) unsigned char smem[];
    void *lut = smem;
    const int Nt = g.Nt;                                  // hidden tiles = down chunks (2 or 3)
    f32x4 *ag_l = (f32x4 *)(smem + lut_bytes<true>());   // [1][4][32]
    f32x4 *au_l = ag_l + 128;
    f32x4 *bg_l = au_l + 128;                             // [Nt][4][32]
    f32x4 *bu_l = bg_l + Nt * 128;
    f32x4 *ad_l = bu_l + Nt * 128;                        // [Nt][4][32] down alpha per chunk
    f32x4 *bd_l = ad_l + Nt * 128;                        // [1][4][32]
    uint2 *areas = (uint2 *)(bd_l + 128);                 // [3][32][64]

    const int tid = threadIdx.x;
    {
        const uint32_t byte = (uint32_t)tid;
        float val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) val[j] = (float)((int)((byte >> (6 - 2 * j)) & 3u) - 1);
        ((uint2 *)lut)[byte] = uint2{pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3])};
    }
    // alpha / beta of the three layers: every load issued before any
    // conversion (buffer loads, zero past the shapes, no branch around them;
    // a conversion or branch right after a load waits for it)
    {
        const __amdgpu_buffer_rsrc_t gar = make_rsrc(g.alpha, (uint32_t)(32 * g.in_o * 4));
        const __amdgpu_buffer_rsrc_t uar = make_rsrc(u.alpha, (uint32_t)(32 * g.in_o * 4));
        const __amdgpu_buffer_rsrc_t dbr = make_rsrc(d.beta, (uint32_t)((31 * d.beta_h + d.out_o) * 4));
        const __amdgpu_buffer_rsrc_t gbr = make_rsrc(g.beta, (uint32_t)(32 * g.out_o * 4));
        const __amdgpu_buffer_rsrc_t ubr = make_rsrc(u.beta, (uint32_t)(32 * g.out_o * 4));
        const __amdgpu_buffer_rsrc_t dar = make_rsrc(d.alpha, (uint32_t)(32 * d.in_o * 4));
        constexpr int kIt = (3 * 128 + kThreads - 1) / kThreads;   // Nt <= 3
        uint32_t r1[3][4], r2[kIt][3][4];
        {
            const int e = tid, gg = e & 31, i0 = 4 * (e >> 5);
            const bool live = e < 128;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool ok = live && i0 + j < g.in_o, okd = live && i0 + j < d.out_o;
                r1[0][j] = __builtin_amdgcn_raw_buffer_load_b32(gar, ok ? (uint32_t)(gg * g.in_o + i0 + j) * 4 : kOOB, 0, 0);
                r1[1][j] = __builtin_amdgcn_raw_buffer_load_b32(uar, ok ? (uint32_t)(gg * g.in_o + i0 + j) * 4 : kOOB, 0, 0);
                r1[2][j] = __builtin_amdgcn_raw_buffer_load_b32(
                    dbr, okd ? (uint32_t)(gg * d.beta_h + i0 + j) * 4 : kOOB, 0, 0);
            }
        }
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int e = tid + it * kThreads, h = e & 31, o0 = 4 * (e >> 5);
            const bool live = e < Nt * 128;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool ok = live && o0 + j < g.out_o, okd = live && o0 + j < d.in_o;
                r2[it][0][j] = __builtin_amdgcn_raw_buffer_load_b32(gbr, ok ? (uint32_t)(h * g.out_o + o0 + j) * 4 : kOOB, 0, 0);
                r2[it][1][j] = __builtin_amdgcn_raw_buffer_load_b32(ubr, ok ? (uint32_t)(h * g.out_o + o0 + j) * 4 : kOOB, 0, 0);
                r2[it][2][j] = __builtin_amdgcn_raw_buffer_load_b32(
                    dar, okd ? (uint32_t)(h * d.in_o + o0 + j) * 4 : kOOB, 0, 0);
            }
        }
        if (tid < 128) {
            const int e = tid, i0 = 4 * (e >> 5);
            f32x4 va, vb, vd;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool ok = i0 + j < g.in_o;
                va[j] = ok ? __uint_as_float(r1[0][j]) : 0.f;
                vb[j] = ok ? __uint_as_float(r1[1][j]) : 0.f;
                vd[j] = i0 + j < d.out_o ? __uint_as_float(r1[2][j]) * 0.03125f : 0.f;
            }
            ag_l[e] = va;
            au_l[e] = vb;
            bd_l[e] = vd;
        }
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int e = tid + it * kThreads, o0 = 4 * (e >> 5);
            if (e >= Nt * 128) continue;
            f32x4 va, vb, vd;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool ok = o0 + j < g.out_o;
                va[j] = ok ? __uint_as_float(r2[it][0][j]) * 0.03125f : 0.f;
                vb[j] = ok ? __uint_as_float(r2[it][1][j]) * 0.03125f : 0.f;
                vd[j] = o0 + j < d.in_o ? __uint_as_float(r2[it][2][j]) : 0.f;  // chunk e / 128, element (h, o0 + j)
            }
            bg_l[e] = va;
            bu_l[e] = vb;
            ad_l[e] = vd;
        }
    }
    __syncthreads();

    const int lane = tid & 63;
    // logical wave: the down wave rotates over the SIMDs with the workgroup
    const int wave = ((tid >> 6) - (int)blockIdx.x) & (kWaves - 1);
    const int t = lane & 15, q = lane >> 4;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.x, (uint32_t)((int64_t)g.M * g.ldx * 2));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(d.y, (uint32_t)((int64_t)d.M * d.ldy * 2));
    const int n_tiles = (int)ceil_div(g.M, kTile);
    for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const int row = tile * kTile + t;
        const bool row_ok = row < g.M;
        if (wave < Nt) {
            const int nt = wave;
            uint2 *st = areas + wave * 32 * 64;
            const uint32_t xoff = (uint32_t)((int64_t)row * g.ldx * 2);
            f32x4 acc[32];
            {   // gate, into the area
                XM<true> xm;
                load_transform<uint16_t, true, true>(g, xr, xoff, row_ok, 0, q, ag_l, xm);
#pragma unroll
                for (int k = 0; k < 32; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
                contract<true>(g, nt, 0, lane, xm, lut, acc);
            }
            fht32x4(acc);
            {
                const f32x4 *bl = bg_l + (nt * 4 + q) * 32;
#pragma unroll
                for (int h0 = 0; h0 < 32; h0 += 4) {
                    f32x4 b4[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) b4[j] = bl[h0 + j];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const f32x4 v = acc[h0 + j] * b4[j];
                        st[(h0 + j) * 64 + lane] = uint2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            {   // up
                XM<true> xm;
                load_transform<uint16_t, true, true>(g, xr, xoff, row_ok, 0, q, au_l, xm);
#pragma unroll
                for (int k = 0; k < 32; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
                contract<true>(u, nt, 0, lane, xm, lut, acc);
            }
            __builtin_amdgcn_sched_barrier(0);
            fht32x4(acc);
            __builtin_amdgcn_sched_barrier(0);
            // h = bf16(silu(g) u) (the SwiGLU kernel's stored value), then
            // the down projection's alpha for chunk nt (zero past hid_o, so
            // those columns contribute zeros, as the down projection's
            // out-of-range loads do)
            {
                const f32x4 *bl = bu_l + (nt * 4 + q) * 32;
                const f32x4 *al = ad_l + (nt * 4 + q) * 32;
#pragma unroll
                for (int h0 = 0; h0 < 32; h0 += 4) {
                    f32x4 b4[4], a4[4];
                    uint2 e4[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        b4[j] = bl[h0 + j];
                        a4[j] = al[h0 + j];
                        e4[j] = st[(h0 + j) * 64 + lane];
                    }
#pragma unroll
                    for (int j4 = 0; j4 < 4; ++j4) {
                        const int h = h0 + j4;
                        const f32x4 uv = acc[h] * b4[j4];
                        const uint2 e = e4[j4];
                        const f32x4 gv{__uint_as_float(e.x << 16), __uint_as_float(e.x & 0xffff0000u),
                                       __uint_as_float(e.y << 16), __uint_as_float(e.y & 0xffff0000u)};
                        f32x4 hv;
#pragma unroll
                        for (int j = 0; j < 4; ++j) hv[j] = silu_fast(gv[j]) * uv[j];
                        const uint32_t p0 = pack_bf16x2(hv.x, hv.y), p1 = pack_bf16x2(hv.z, hv.w);
                        const f32x4 hb{__uint_as_float(p0 << 16), __uint_as_float(p0 & 0xffff0000u),
                                       __uint_as_float(p1 << 16), __uint_as_float(p1 & 0xffff0000u)};
                        acc[h] = hb * a4[j4];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            fht32x4(acc);
            __builtin_amdgcn_sched_barrier(0);
            // the transformed chunk replaces the gate stash (this wave's own
            // area: its reads above are done, LDS operations run in order)
            wave_lds_fence();
#pragma unroll
            for (int h = 0; h < 32; ++h)
                st[h * 64 + lane] = uint2{pack_bf16x2(acc[h].x, acc[h].y), pack_bf16x2(acc[h].z, acc[h].w)};
            lds_barrier();  // A: the chunks are in the areas
            lds_barrier();  // B: the down wave has read them
        } else if (wave == kMlpDownWave) {
            lds_barrier();  // A
            f32x4 acc[32];
#pragma unroll
            for (int k = 0; k < 32; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
            for (int c = 0; c < Nt; ++c) {
                XM<true> xm;
                const uint2 *st = areas + c * 32 * 64;
#pragma unroll
                for (int h = 0; h < 32; ++h) xm.b[h] = st[h * 64 + lane];
                contract<true>(d, 0, c, lane, xm, lut, acc);
            }
            lds_barrier();  // B
            transform_store<uint16_t, true>(d, acc, yr, (uint32_t)((int64_t)row * d.ldy * 2), row_ok, 0, q, bd_l,
                                            row);
        } else {
            lds_barrier();  // A
            lds_barrier();  // B
        }
    }
}

// ---------------------------------------------------------------- standalone FHT
// Normalised (or not) fast Walsh-Hadamard transform of rows of length
// N = 2^logN (fht_cuda.py:281-309): rows staged in LDS, log2(N) butterfly
// stages (k, k + h) -> (a + b, a - b) separated by barriers.
template <typename T>
__global__ __launch_bounds__(256) void fht_kernel(const T *__restrict__ x, int64_t rows, int logN, float scale,
                                                  T *__restrict__ y) {
    extern __shared__ float buf[];
    const int N = 1 << logN;
    const int rpb = N >= 4096 ? 1 : 4096 / N;
    const int64_t row0 = (int64_t)blockIdx.x * rpb;
    const int nr = (int)((rows - row0) < rpb ? (rows - row0) : rpb);
    const int tot = nr * N;
    for (int e = threadIdx.x; e < tot; e += blockDim.x) buf[e] = Act<T>::load(x + row0 * N + e);
    __syncthreads();
    const int half = N / 2;
    for (int h = 1; h < N; h <<= 1) {
        for (int p = threadIdx.x; p < nr * half; p += blockDim.x) {
            const int r = p / half, j = p - r * half;
            const int i = (j / h) * 2 * h + (j % h);
            float *row = buf + r * N;
            const float a = row[i], b = row[i + h];
            row[i] = a + b;
            row[i + h] = a - b;
        }
        __syncthreads();
    }
    for (int e = threadIdx.x; e < tot; e += blockDim.x) Act<T>::store(y + row0 * N + e, buf[e] * scale);
}

// Dense weights as A fragments [Nt][Kc][32 g][64 lanes] x 4 values: lane l
// of (nt, c) holds for group g the weights W[g, o, i..i+3] with
// o = 16nt + l%16, i = 16c + 4(l/16) (0 past out_o / in_o).  w_io: the
// source is stored [32][in_o][out_o] (the head mixer's x @ W) instead of
// [32][out_o][in_o].
// Wide layout (bf16 with 32 < in_o <= 128, out_o <= 128: the wide kernel's
// 16x16x32 products): [Nt][in_o/32][32 g][64 lanes] x 8 values, lane l of
// (nt, c) holding W[g, 16nt + l%16, 32c + 8(l/16) .. +7].
__global__ void hadamard_dense_prepare32_kernel(const float *__restrict__ w, int in_o, int out_o, int w_io, int Nt,
                                                int Kc32, uint4 *__restrict__ kw) {
    const int64_t total = (int64_t)Nt * Kc32 * 32 * 64;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(e & 63);
        const int g = (int)((e >> 6) & 31);
        const int64_t tc = e >> 11;
        const int c = (int)(tc % Kc32);
        const int nt = (int)(tc / Kc32);
        const int o = kNTile * nt + (lane & 15);
        const int i0 = 32 * c + 8 * (lane >> 4);
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j;
            v[j] = (o < out_o && i < in_o)
                       ? w[w_io ? ((int64_t)g * in_o + i) * out_o + o : ((int64_t)g * out_o + o) * in_o + i]
                       : 0.f;
        }
        kw[e] = uint4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                      pack_bf16x2(v[6], v[7])};
    }
}

__global__ void hadamard_dense_prepare_kernel(const float *__restrict__ w, int in_o, int out_o, int w_io, int Nt,
                                              int Kc, int bf16, unsigned char *__restrict__ kw) {
    const int64_t total = (int64_t)Nt * Kc * 32 * 64;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(e & 63);
        const int g = (int)((e >> 6) & 31);
        const int64_t tc = e >> 11;
        const int c = (int)(tc % Kc);
        const int nt = (int)(tc / Kc);
        const int o = kNTile * nt + (lane & 15);
        const int i0 = kKChunk * c + 4 * (lane >> 4);
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = i0 + j;
            v[j] = (o < out_o && i < in_o)
                       ? w[w_io ? ((int64_t)g * in_o + i) * out_o + o : ((int64_t)g * out_o + o) * in_o + i]
                       : 0.f;
        }
        if (bf16)
            ((uint2 *)kw)[e] = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        else
            ((f32x4 *)kw)[e] = f32x4{v[0], v[1], v[2], v[3]};
    }
}

static size_t hadamard_lds_bytes(bool bf16, int Kc, int Nt) {
    return (bf16 ? lut_bytes<true>() : lut_bytes<false>()) + (size_t)16 * 128 * (Kc + Nt);
}

}  // namespace walsh

using namespace walsh;

// Shapes that also get the base-3 layout of the wide bf16 kernel.
static bool wide3_shape(int64_t in_o, int64_t out_o) {
    return in_o > kKChunk && in_o <= kW3MaxO && out_o <= kW3MaxO;
}

static int64_t weight_bytes1(int64_t in_o, int64_t out_o) {
    return ceil_div(out_o, kNTile) * ceil_div(in_o, kKChunk) * 64 * 32;
}

// The first layout, followed by the base-3 one for wide3_shape.
WALSH_EXPORT int64_t walsh_hadamard_weight_bytes(int64_t in_o, int64_t out_o) {
    if (in_o <= 0 || out_o <= 0) return 0;
    int64_t n = weight_bytes1(in_o, out_o);
    if (wide3_shape(in_o, out_o)) n += ceil_div(out_o, kNTile) * ceil_div(in_o, 32) * 4096;
    return n;
}

WALSH_EXPORT int walsh_hadamard_prepare(const uint8_t *packed, int64_t in_o, int64_t out_o, uint8_t *kweight,
                                        void *stream) {
    if (!packed || !kweight) return set_error(WALSH_EINVAL, "walsh_hadamard_prepare: null pointer");
    if (in_o <= 0 || out_o <= 0 || in_o > (1 << 20) || out_o > (1 << 20))
        return set_error(WALSH_EINVAL, "walsh_hadamard_prepare: bad shape in_o=%lld out_o=%lld", (long long)in_o,
                         (long long)out_o);
    const int Nt = (int)ceil_div(out_o, kNTile), Kc = (int)ceil_div(in_o, kKChunk);
    const int64_t total = (int64_t)Nt * Kc * 2048;
    const int block = 256;
    int grid = (int)ceil_div(total, block);
    if (grid > 4096) grid = 4096;
    launch(hadamard_prepare_kernel, dim3(grid), dim3(block), 0, (hipStream_t)stream, packed, (int)in_o,
                       (int)out_o, Nt, Kc, kweight);
    if (wide3_shape(in_o, out_o)) {
        const int Kc32 = (int)ceil_div(in_o, 32);
        const int64_t total3 = (int64_t)Nt * Kc32 * 4096;
        int grid3 = (int)ceil_div(total3, block);
        if (grid3 > 4096) grid3 = 4096;
        launch(hadamard_prepare3_kernel, dim3(grid3), dim3(block), 0, (hipStream_t)stream, packed, (int)in_o,
               (int)out_o, Nt, Kc32, kweight + weight_bytes1(in_o, out_o));
    }
    return check_hip(hipGetLastError(), "walsh_hadamard_prepare launch");
}

static int hadamard_check(const char *fn, const void *x, int64_t ldx, int64_t gsx, int64_t M, int64_t in_o,
                          int64_t out_o, const void *y, int64_t ldy, int64_t gsy, int dtype) {
    if (!x || !y) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || in_o <= 0 || out_o <= 0 || in_o > 65536 || out_o > 65536)
        return set_error(WALSH_EINVAL, "%s: bad shape M=%lld in_o=%lld out_o=%lld", fn, (long long)M, (long long)in_o,
                         (long long)out_o);
    if (gsx < in_o || gsy < out_o || ldx < 32 * gsx || ldy < 32 * gsy)
        return set_error(WALSH_EINVAL, "%s: strides too small (ldx=%lld gsx=%lld ldy=%lld gsy=%lld)", fn,
                         (long long)ldx, (long long)gsx, (long long)ldy, (long long)gsy);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d not supported", fn, dtype);
    return WALSH_OK;
}

// Launch one Hadamard-linear (two for the fused SwiGLU: u != NULL) over M
// rows in chunks whose byte offsets fit a 31-bit buffer range.
// hadamard_pair_kernel over rows rows of an.n layers: one workgroup (a
// wavefront pair) per 16-row tile and layer, up to the workgroups the CUs
// hold at once (LDS: kPairLds each; registers: 4 wavefronts per SIMD), the
// rest looped over.
static void pair_launch(const HadArgsN &an, int64_t rows, hipStream_t s, bool dense = false) {
    const int64_t per_cu = (int64_t)device_info().lds_per_cu / (int64_t)kPairLds;
    const int64_t by_regs = dense ? 6 : 8;   // 3 or 4 wavefronts per SIMD
    const int64_t resident = (int64_t)device_info().cu_count * (per_cu < by_regs ? per_cu : by_regs);
    int64_t per_layer = ceil_div(rows, kTile);
    const int64_t cap = resident / an.n > 0 ? resident / an.n : 1;
    if (per_layer > cap) per_layer = cap;
    const dim3 G((unsigned)(per_layer * an.n)), B(kPairThreads);
    if (dense) launch(hadamard_pair_kernel<true>, G, B, (uint32_t)kPairLds, s, an);
    else launch(hadamard_pair_kernel<false>, G, B, (uint32_t)kPairLds, s, an);
}

static void pair_kpar_launch(const HadArgs &a, int64_t rows, hipStream_t s) {
    // chunk-parallel: Kc wavefront pairs per tile, as many workgroups as the
    // CUs hold at once (LDS: kpar_lds each; registers: 3 wavefronts per SIMD)
    const size_t lds = kpar_lds(a.Kc);
    int64_t per_cu = (int64_t)device_info().lds_per_cu / (int64_t)lds;
    const int64_t by_regs = 12 / (2 * (int64_t)a.Kc);
    if (per_cu > by_regs) per_cu = by_regs;
    if (per_cu < 1) per_cu = 1;
    int64_t grid = ceil_div(rows, kTile);
    const int64_t resident = (int64_t)device_info().cu_count * per_cu;
    if (grid > resident) grid = resident;
    launch(hadamard_pair_kpar_kernel, dim3((unsigned)grid), dim3(kPairThreads * a.Kc), (uint32_t)lds, s, a);
}

static int hadamard_launch(const char *fn, HadArgs base, const HadArgs *ubase, int64_t M, bool bf16, hipStream_t s) {
    const int64_t esz = bf16 ? 2 : 4;
    const int Nt = base.Nt, Kc = base.Kc;
    const bool swiglu = ubase != nullptr;
    size_t lds = hadamard_lds_bytes(bf16, Kc, Nt);
    // SwiGLU: the up projection's alpha / beta tables and, per working wave,
    // the gate output (32 groups x 64 lanes x 4 values)
    const size_t stash_wave = (size_t)32 * 64 * (bf16 ? 8 : 16);
    if (swiglu) lds += (size_t)16 * 128 * (Kc + Nt);
    if (lds + (swiglu ? kWaves * stash_wave : 0) > (size_t)device_info().max_shared_per_block)
        return set_error(WALSH_ENOTSUP, "%s: in_o=%d out_o=%d need %zu B of LDS", fn, base.in_o, base.out_o,
                         lds + (swiglu ? kWaves * stash_wave : 0));
    const size_t valign = bf16 ? 8 : 16;
    const bool vec = (base.gsx % 4 == 0) && (base.ldx % 4 == 0) && ((uintptr_t)base.x % valign == 0) &&
                     (base.gsy % 4 == 0) && (base.ldy % 4 == 0) && ((uintptr_t)base.y % valign == 0);
    // float32 operands keep 128 registers of transformed input; with several
    // output tiles they are recomputed per tile instead of kept live.
    const bool kc1 = Kc == 1 && (bf16 || Nt == 1);
    // several input chunks and output tiles: the workgroup-wide kernel
    const size_t wide_lds = bf16 ? wide_lds_bytes<true>() : wide_lds_bytes<false>();
    const bool wide = !swiglu && vec && Kc >= 2 && Nt >= 4 && wide_lds <= (size_t)device_info().max_shared_per_block;
    // bf16 with in_o <= 128 and out_o <= 128: the base-3 16x16x32 kernel
    const size_t wide3_lds = wide3_lds_bytes((base.in_o + 31) / 32);
    const bool wide3 = wide && bf16 && base.kw3 != nullptr && wide3_lds <= (size_t)device_info().max_shared_per_block;
    const int64_t ld = base.ldx > base.ldy ? base.ldx : base.ldy;
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * esz);
    rows_max = rows_max / kTile * kTile;
    if (rows_max < kTile) return set_error(WALSH_ENOTSUP, "%s: row stride too large", fn);
    rows_max = balanced_rows(M, rows_max, kTile);
    const int64_t cap = (int64_t)device_info().cu_count * (swiglu ? 8 : 2);
    // rows of exactly 512 contiguous bf16 on both sides (every chunk keeps
    // the 16-byte alignment): the one-wavefront kernel's STAGED variant
    const size_t st_lds_max = lds + (size_t)kWaves * kStageBytes;
    const bool whole_rows = !swiglu && bf16 && vec && kc1 && Nt == 1 && base.in_o == 16 && base.out_o == 16 &&
                            base.gsx == 16 && base.gsy == 16 && base.ldx == 512 && base.ldy == 512 && base.tpb == 0 &&
                            (uintptr_t)base.x % 16 == 0 && (uintptr_t)base.y % 16 == 0 &&
                            st_lds_max <= (size_t)device_info().max_shared_per_block;
    const int64_t pair_max = whole_rows ? kPairMaxTilesRows : kPairMaxTiles;
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        HadArgs a = base;
        a.x = (const char *)base.x + r0 * base.ldx * esz;
        a.rope_row0 = (int)(r0 % base.rope_T);
        a.y = (char *)base.y + r0 * base.ldy * esz;
        a.M = (int)rows;
        int64_t work = ceil_div(rows, kTile) * (swiglu ? Nt : 1);
        int64_t grid = ceil_div(work, kWaves);
        // workgroups per CU these bf16 variants hold (register-bound: two for
        // one input chunk, one for the chunk loop)
        const int64_t resident = (int64_t)device_info().cu_count * (Kc == 1 ? 2 : 1);
        if (vec && bf16 && work <= resident * kWaves) {
            // all the work fits in one residency round of this variant: give
            // each workgroup ceil(work / resident) working waves, so every CU
            // holds the same number of them
            const int64_t wt = ceil_div(work, resident);
            a.wave_tiles = (int)wt;
            grid = ceil_div(work, wt);
        }
        // the single-chunk SwiGLU kernel holds two workgroups per CU by its
        // registers; with a stash for each of 4 waves its LDS would allow
        // one, so 3 of its waves take items and the stash is sized for them
        if (swiglu && Kc == 1 && (a.wave_tiles <= 0 || a.wave_tiles > 3)) {
            a.wave_tiles = 3;
            grid = ceil_div(work, 3);
            if (grid > resident) grid = resident;   // one round; waves loop over the rest
        }
        if (grid > cap) grid = cap;
        const dim3 G((unsigned)grid), B(kThreads);
        if (swiglu) {
            HadArgs ua = *ubase;
            ua.x = a.x;
            ua.y = a.y;
            ua.M = a.M;
            ua.wave_tiles = a.wave_tiles;
            const size_t sw_lds = lds + (size_t)(a.wave_tiles > 0 ? a.wave_tiles : kWaves) * stash_wave;
#define WALSH_SW_LAUNCH(T, MMA, V, K1) launch((hadamard_swiglu_kernel<T, MMA, V, K1>), G, B, sw_lds, s, a, ua)
            const bool one = Kc == 1;
            if (bf16) {
                if (vec) { if (one) WALSH_SW_LAUNCH(uint16_t, true, true, true); else WALSH_SW_LAUNCH(uint16_t, true, true, false); }
                else     { if (one) WALSH_SW_LAUNCH(uint16_t, true, false, true); else WALSH_SW_LAUNCH(uint16_t, true, false, false); }
            } else {
                if (vec) { if (one) WALSH_SW_LAUNCH(float, false, true, true); else WALSH_SW_LAUNCH(float, false, true, false); }
                else     { if (one) WALSH_SW_LAUNCH(float, false, false, true); else WALSH_SW_LAUNCH(float, false, false, false); }
            }
#undef WALSH_SW_LAUNCH
        } else if (wide3 && rows <= kSplitRows) {
            HadArgsN an;
            an.n = 1;
            an.p[0] = a;
            split3_launch(an, a.gsx == 128 && a.gsy == 128 && a.in_o == 128 && a.out_o == 128, false, s);
        } else if (wide3) {
            const int64_t items = ceil_div(rows, kTile);
            const int64_t wcap = (int64_t)device_info().cu_count;
            const dim3 G3((unsigned)(items < wcap ? items : wcap)), B3(kWideThreads);
            if (a.gsx == 128 && a.gsy == 128 && a.in_o == 128 && a.out_o == 128)
                launch(hadamard_wide3_kernel<128>, G3, B3, wide3_lds, s, a);
            else launch(hadamard_wide3_kernel<0>, G3, B3, wide3_lds, s, a);
        } else if (wide) {
            const int64_t items = ceil_div(rows, kTile) * ceil_div(Nt, kWideWaves);
            const int64_t wcap = (int64_t)device_info().cu_count;
            const dim3 GW((unsigned)(items < wcap ? items : wcap)), BW(kWideThreads);
            const bool a4 = base.in_o % 2 == 0;
            if (bf16) {
                if (a4) launch((hadamard_wide_kernel<uint16_t, true, true>), GW, BW, wide_lds, s, a);
                else launch((hadamard_wide_kernel<uint16_t, true, false>), GW, BW, wide_lds, s, a);
            } else {
                if (a4) launch((hadamard_wide_kernel<float, false, true>), GW, BW, wide_lds, s, a);
                else launch((hadamard_wide_kernel<float, false, false>), GW, BW, wide_lds, s, a);
            }
        } else if (bf16 && vec && Nt == 1 && Kc > 1 && Kc <= kPairMaxKc && !base.rope &&
                   ceil_div(rows, kTile) <= kPairMaxTiles) {
            // several input chunks, one output tile: a wavefront pair per tile
            pair_kpar_launch(a, rows, s);
        } else if (bf16 && vec && kc1 && Nt == 1 && ceil_div(rows, kTile) <= pair_max) {
            // one input chunk, one output tile, up to pair_max tiles: a
            // wavefront pair per tile
            HadArgsN an;
            an.n = 1;
            an.p[0] = a;
            pair_launch(an, rows, s);
        } else {
#define WALSH_HAD_LAUNCH(T, MMA, V, K1) launch((hadamard_fwd_kernel<T, MMA, V, K1>), G, B, lds, s, a)
            if (bf16) {
                // whole 1 KB rows on both sides: through the per-wave LDS areas
                const size_t st_lds = lds + (size_t)(a.wave_tiles > 0 ? a.wave_tiles : kWaves) * kStageBytes;
                a.nt_store = rows * 1024 >= kStreamOutBytes;
                if (whole_rows) launch((hadamard_fwd_kernel<uint16_t, true, true, true, false, true, true>), G, B, st_lds, s, a);
                else if (vec && kc1 && Nt == 1) launch((hadamard_fwd_kernel<uint16_t, true, true, true, false, true>), G, B, lds, s, a);
                else if (vec) { if (kc1) WALSH_HAD_LAUNCH(uint16_t, true, true, true); else WALSH_HAD_LAUNCH(uint16_t, true, true, false); }
                else     { if (kc1) WALSH_HAD_LAUNCH(uint16_t, true, false, true); else WALSH_HAD_LAUNCH(uint16_t, true, false, false); }
            } else {
                if (vec) { if (kc1) WALSH_HAD_LAUNCH(float, false, true, true); else WALSH_HAD_LAUNCH(float, false, true, false); }
                else     { if (kc1) WALSH_HAD_LAUNCH(float, false, false, true); else WALSH_HAD_LAUNCH(float, false, false, false); }
            }
#undef WALSH_HAD_LAUNCH
        }
        const int rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
    }
    return WALSH_OK;
}

static HadArgs had_args(const void *x, int64_t ldx, int64_t gsx, int64_t in_o, int64_t out_o, const uint8_t *kw,
                        const float *alpha, const float *beta, void *y, int64_t ldy, int64_t gsy) {
    HadArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.M = 0;
    a.in_o = (int)in_o;
    a.out_o = (int)out_o;
    a.Nt = (int)ceil_div(out_o, kNTile);
    a.Kc = (int)ceil_div(in_o, kKChunk);
    a.gsx = (int)gsx;
    a.gsy = (int)gsy;
    a.kw = kw;
    a.kw3 = wide3_shape(in_o, out_o) ? kw + weight_bytes1(in_o, out_o) : nullptr;
    a.alpha = alpha;
    a.beta = beta;
    a.beta_h = (int)out_o;
    a.y = y;
    a.ldy = ldy;
    a.tpb = 0;
    a.bstride = 0;
    a.xspan = 0;
    a.rope = nullptr;
    a.rope_T = 1;
    a.rope_D = 4;
    a.rope_row0 = 0;
    a.wave_tiles = 0;
    return a;
}

WALSH_EXPORT int walsh_hadamard_linear_ex_fwd(const void *x, int64_t ldx, int64_t gsx, int64_t M, int64_t in_o,
                                              int64_t out_o, const uint8_t *kweight, const float *alpha,
                                              const float *beta, void *y, int64_t ldy, int64_t gsy, int dtype,
                                              void *stream) {
    const char *fn = "walsh_hadamard_linear_ex_fwd";
    int rc = hadamard_check(fn, x, ldx, gsx, M, in_o, out_o, y, ldy, gsy, dtype);
    if (rc) return rc;
    if (!kweight || !alpha || !beta) return set_error(WALSH_EINVAL, "%s: null weight pointer", fn);
    if (M == 0) return WALSH_OK;
    return hadamard_launch(fn, had_args(x, ldx, gsx, in_o, out_o, kweight, alpha, beta, y, ldy, gsy), nullptr, M,
                           dtype == WALSH_BF16, (hipStream_t)stream);
}

WALSH_EXPORT int walsh_hadamard_linear_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                                           const uint8_t *kweight, const float *alpha, const float *beta, void *y,
                                           int64_t ldy, int dtype, void *stream) {
    return walsh_hadamard_linear_ex_fwd(x, ldx, in_o, M, in_o, out_o, kweight, alpha, beta, y, ldy, out_o, dtype,
                                        stream);
}

WALSH_EXPORT int walsh_hadamard_linear_rope_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                                                const uint8_t *kweight, const float *alpha, const float *beta,
                                                const float *rope, int64_t rope_T, int64_t head_dim, void *y,
                                                int64_t ldy, int dtype, void *stream) {
    const char *fn = "walsh_hadamard_linear_rope_fwd";
    int rc = hadamard_check(fn, x, ldx, in_o, M, in_o, out_o, y, ldy, out_o, dtype);
    if (rc) return rc;
    if (!kweight || !alpha || !beta || !rope) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (rope_T < 1 || head_dim < 4 || head_dim % 4 || out_o % head_dim || (uintptr_t)rope % 16)
        return set_error(WALSH_ENOTSUP, "%s: needs head_dim %% 4 == 0 dividing out_o, 16-byte aligned table", fn);
    const size_t valign = dtype == WALSH_BF16 ? 8 : 16;
    if (ldx % 4 || ldy % 4 || in_o % 4 || (uintptr_t)x % valign || (uintptr_t)y % valign)
        return set_error(WALSH_ENOTSUP, "%s: needs 4-aligned rows and in_o", fn);
    if (M == 0) return WALSH_OK;
    HadArgs a = had_args(x, ldx, in_o, in_o, out_o, kweight, alpha, beta, y, ldy, out_o);
    a.rope = rope;
    a.rope_T = (int)rope_T;
    a.rope_D = (int)head_dim;
    return hadamard_launch(fn, a, nullptr, M, dtype == WALSH_BF16, (hipStream_t)stream);
}

static int hadamard_multi(const char *fn, const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                          int64_t n, const uint8_t *const *kweights, const float *const *alphas,
                          const float *const *betas, void *const *ys, const int64_t *ldys, const int64_t *gsys,
                          const float *rope, int64_t rope_T, int64_t head_dim, int rope_mask, int dtype, void *stream) {
    if (n < 1 || n > kMaxMulti || !kweights || !alphas || !betas || !ys || !ldys || !gsys)
        return set_error(WALSH_EINVAL, "%s: n=%lld (1..%d) or null array", fn, (long long)n, kMaxMulti);
    if (rope_mask & ~((1 << n) - 1)) return set_error(WALSH_EINVAL, "%s: rope_mask 0x%x past n", fn, rope_mask);
    HadArgs base[kMaxMulti];
    for (int i = 0; i < n; ++i) {
        int rc = hadamard_check(fn, x, ldx, in_o, M, in_o, out_o, ys[i], ldys[i], gsys[i], dtype);
        if (rc) return rc;
        if (!kweights[i] || !alphas[i] || !betas[i]) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
        base[i] = had_args(x, ldx, in_o, in_o, out_o, kweights[i], alphas[i], betas[i], ys[i], ldys[i], gsys[i]);
        if (rope_mask & (1 << i)) {
            if (!rope || rope_T < 1 || head_dim < 4 || head_dim % 4 || out_o % head_dim || (uintptr_t)rope % 16)
                return set_error(WALSH_ENOTSUP, "%s: RoPE needs head_dim %% 4 == 0 dividing out_o, 16-byte aligned "
                                 "table", fn);
            base[i].rope = rope;
            base[i].rope_T = (int)rope_T;
            base[i].rope_D = (int)head_dim;
        }
    }
    if (M == 0) return WALSH_OK;
    const bool bf16 = dtype == WALSH_BF16;
    const int64_t esz = bf16 ? 2 : 4;
    const size_t valign = bf16 ? 8 : 16;
    const int Nt = base[0].Nt, Kc = base[0].Kc;
    bool vec = in_o % 4 == 0 && out_o % 4 == 0 && ldx % 4 == 0 && (uintptr_t)x % valign == 0;
    int64_t ldy = 0;  // the longest output row stride
    bool gs128 = in_o == 128 && out_o == 128;
    for (int i = 0; i < n; ++i) {
        vec = vec && (uintptr_t)ys[i] % valign == 0 && ldys[i] % 4 == 0 && gsys[i] % 4 == 0;
        gs128 = gs128 && gsys[i] == 128;
        if (ldys[i] > ldy) ldy = ldys[i];
    }
    const bool kc1 = Kc == 1 && (bf16 || Nt == 1);
    const size_t lds = hadamard_lds_bytes(bf16, Kc, Nt);
    hipStream_t s = (hipStream_t)stream;
    const int64_t ld = ldx > ldy ? ldx : ldy;
    if (bf16 && vec && base[0].kw3 && Kc >= 2 && Nt >= 4 && M <= kSplitRows &&
        M * ld * esz <= (int64_t)kMaxBufferBytes &&
        split3_lds_bytes((int)ceil_div(in_o, 32)) <= (size_t)device_info().max_shared_per_block) {
        // a few rows of a wide3 shape: every layer in one split launch
        HadArgsN an;
        an.n = (int)n;
        for (int i = 0; i < n; ++i) {
            an.p[i] = base[i];
            an.p[i].M = (int)M;
        }
        split3_launch(an, gs128, false, s);
        return check_hip(hipGetLastError(), fn);
    }
    bool gs_plain = true;  // the one-launch kernel for small in_o writes packed groups
    for (int i = 0; i < n; ++i) gs_plain = gs_plain && gsys[i] == out_o;
    if (!kc1 || !vec || !gs_plain || lds > (size_t)device_info().max_shared_per_block) {
        // shapes served by the other kernels: one launch per layer
        for (int i = 0; i < n; ++i) {
            const int rc = hadamard_launch(fn, base[i], nullptr, M, bf16, s);
            if (rc) return rc;
        }
        return WALSH_OK;
    }
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * esz) / kTile * kTile;
    if (rows_max < kTile) return set_error(WALSH_ENOTSUP, "%s: row stride too large", fn);
    rows_max = balanced_rows(M, rows_max, kTile);
    const int64_t cap = (int64_t)device_info().cu_count * 2;
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        HadArgsN an;
        an.n = (int)n;
        for (int i = 0; i < n; ++i) {
            an.p[i] = base[i];
            an.p[i].x = (const char *)x + r0 * ldx * esz;
            an.p[i].y = (char *)ys[i] + r0 * ldys[i] * esz;
            an.p[i].M = (int)rows;
            an.p[i].rope_row0 = (int)(r0 % base[i].rope_T);
        }
        int64_t grid = ceil_div(ceil_div(rows, kTile), kWaves);
        if (grid > cap) grid = cap;
        const dim3 G((unsigned)(grid * n)), B(kThreads);
        // whole 1 KB rows on both sides of every layer: through per-wave LDS areas
        const size_t st_lds = lds + (size_t)kWaves * kStageBytes;
        bool staged = bf16 && Nt == 1 && in_o == 16 && out_o == 16 && ldx == 512 && (uintptr_t)an.p[0].x % 16 == 0 &&
                      st_lds <= (size_t)device_info().max_shared_per_block;
        for (int i = 0; i < n; ++i) {
            staged = staged && base[i].tpb == 0 && ldys[i] == 512 && (uintptr_t)an.p[i].y % 16 == 0;
            an.p[i].nt_store = rows * 1024 >= kStreamOutBytes;
        }
        if (bf16 && Nt == 1 && ceil_div(rows, kTile) <= (staged ? kPairMaxTilesRows : kPairMaxTiles))
            pair_launch(an, rows, s);
        else if (staged) launch((hadamard_fwdn_kernel<uint16_t, true, true, true, true, true>), G, B, st_lds, s, an);
        else if (bf16 && Nt == 1) launch((hadamard_fwdn_kernel<uint16_t, true, true, true, true>), G, B, lds, s, an);
        else if (bf16) launch((hadamard_fwdn_kernel<uint16_t, true, true, true>), G, B, lds, s, an);
        else launch((hadamard_fwdn_kernel<float, false, true, true>), G, B, lds, s, an);
        const int rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
    }
    return WALSH_OK;
}

WALSH_EXPORT int walsh_hadamard_linear_multi_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t out_o,
                                                 int64_t n, const uint8_t *const *kweights, const float *const *alphas,
                                                 const float *const *betas, void *const *ys, int64_t ldy,
                                                 const float *rope, int64_t rope_T, int64_t head_dim, int rope_mask,
                                                 int dtype, void *stream) {
    int64_t ldys[kMaxMulti], gsys[kMaxMulti];
    for (int i = 0; i < kMaxMulti; ++i) {
        ldys[i] = ldy;
        gsys[i] = out_o;
    }
    return hadamard_multi("walsh_hadamard_linear_multi_fwd", x, ldx, M, in_o, out_o, n, kweights, alphas, betas, ys,
                          ldys, gsys, rope, rope_T, head_dim, rope_mask, dtype, stream);
}

WALSH_EXPORT int walsh_hadamard_linear_multi_ex_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o,
                                                    int64_t out_o, int64_t n, const uint8_t *const *kweights,
                                                    const float *const *alphas, const float *const *betas,
                                                    void *const *ys, const int64_t *ldys, const int64_t *gsys,
                                                    const float *rope, int64_t rope_T, int64_t head_dim,
                                                    int rope_mask, int dtype, void *stream) {
    return hadamard_multi("walsh_hadamard_linear_multi_ex_fwd", x, ldx, M, in_o, out_o, n, kweights, alphas, betas,
                          ys, ldys, gsys, rope, rope_T, head_dim, rope_mask, dtype, stream);
}

WALSH_EXPORT int walsh_hadamard_swiglu_fwd(const void *x, int64_t ldx, int64_t gsx, int64_t M, int64_t in_o,
                                           int64_t hid_o, const uint8_t *kw_gate, const float *alpha_gate,
                                           const float *beta_gate, const uint8_t *kw_up, const float *alpha_up,
                                           const float *beta_up, void *h, int64_t ldh, int64_t gsh, int dtype,
                                           void *stream) {
    const char *fn = "walsh_hadamard_swiglu_fwd";
    int rc = hadamard_check(fn, x, ldx, gsx, M, in_o, hid_o, h, ldh, gsh, dtype);
    if (rc) return rc;
    if (!kw_gate || !alpha_gate || !beta_gate || !kw_up || !alpha_up || !beta_up)
        return set_error(WALSH_EINVAL, "%s: null weight pointer", fn);
    if (M == 0) return WALSH_OK;
    const HadArgs ga = had_args(x, ldx, gsx, in_o, hid_o, kw_gate, alpha_gate, beta_gate, h, ldh, gsh);
    const HadArgs ua = had_args(x, ldx, gsx, in_o, hid_o, kw_up, alpha_up, beta_up, h, ldh, gsh);
    return hadamard_launch(fn, ga, &ua, M, dtype == WALSH_BF16, (hipStream_t)stream);
}

WALSH_EXPORT int walsh_hadamard_mlp_fwd(const void *x, int64_t ldx, int64_t M, int64_t in_o, int64_t hid_o,
                                       int64_t out_o, const uint8_t *kw_gate, const float *alpha_gate,
                                       const float *beta_gate, const uint8_t *kw_up, const float *alpha_up,
                                       const float *beta_up, const uint8_t *kw_down, const float *alpha_down,
                                       const float *beta_down, void *y, int64_t ldy, int dtype, void *stream) {
    const char *fn = "walsh_hadamard_mlp_fwd";
    if (!x || !y || !kw_gate || !alpha_gate || !beta_gate || !kw_up || !alpha_up || !beta_up || !kw_down ||
        !alpha_down || !beta_down)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (dtype != WALSH_BF16 || in_o < 1 || in_o > kKChunk || in_o % 4 || hid_o <= kNTile || hid_o > 3 * kNTile ||
        out_o < 1 || out_o > kNTile || out_o % 4)
        return set_error(WALSH_ENOTSUP, "%s: needs bf16, in_o <= 16 and out_o <= 16 (multiples of 4), 16 < hid_o <= 48 "
                         "(got in_o=%lld hid_o=%lld out_o=%lld)", fn, (long long)in_o, (long long)hid_o,
                         (long long)out_o);
    if (M < 0 || ldx < 32 * in_o || ldy < 32 * out_o || ldx % 4 || ldy % 4 || (uintptr_t)x % 8 || (uintptr_t)y % 8)
        return set_error(WALSH_EINVAL, "%s: bad rows (M=%lld ldx=%lld ldy=%lld; rows 8-byte aligned, strides "
                         "multiples of 4)", fn, (long long)M, (long long)ldx, (long long)ldy);
    if (M == 0) return WALSH_OK;
    HadArgs ga = had_args(x, ldx, in_o, in_o, hid_o, kw_gate, alpha_gate, beta_gate, nullptr, 0, hid_o);
    HadArgs ua = had_args(x, ldx, in_o, in_o, hid_o, kw_up, alpha_up, beta_up, nullptr, 0, hid_o);
    HadArgs da = had_args(nullptr, 0, hid_o, hid_o, out_o, kw_down, alpha_down, beta_down, y, ldy, out_o);
    const int Nt = ga.Nt;
    const size_t lds = lut_bytes<true>() + (size_t)16 * 128 * (2 + 3 * Nt + 1) + (size_t)3 * 32 * 64 * 8;
    if (lds > (size_t)device_info().max_shared_per_block)
        return set_error(WALSH_ENOTSUP, "%s: needs %zu B of LDS", fn, lds);
    const int64_t ld = ldx > ldy ? ldx : ldy;
    const int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * 2) / kTile * kTile;
    const int64_t resident = (int64_t)device_info().cu_count * 2;
    hipStream_t s = (hipStream_t)stream;
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        HadArgs g = ga, u = ua, d = da;
        g.x = u.x = (const char *)x + r0 * ldx * 2;
        d.y = (char *)y + r0 * ldy * 2;
        g.M = u.M = d.M = (int)rows;
        int64_t grid = ceil_div(rows, kTile);
        if (grid > resident) grid = resident;
        launch(hadamard_mlp_kernel, dim3((unsigned)grid), dim3(kThreads), (uint32_t)lds, s, g, u, d);
        const int rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
    }
    return WALSH_OK;
}

// ---------------------------------------------------------------- head mixer

constexpr int kDenseMaxO = 32;  // head_dim limit of the LDS-resident dense path

// bf16 shapes that take the wide kernel (weights streamed from memory)
static bool dense_wide(int64_t in_o, int64_t out_o, int dtype) {
    return dtype == WALSH_BF16 && in_o > kDenseMaxO && in_o <= kW3MaxO && out_o > kDenseMaxO && out_o <= kW3MaxO;
}

WALSH_EXPORT int64_t walsh_hadamard_dense_weight_bytes(int64_t in_o, int64_t out_o, int dtype) {
    if (in_o <= 0 || out_o <= 0 || (dtype != WALSH_F32 && dtype != WALSH_BF16)) return 0;
    if (dense_wide(in_o, out_o, dtype)) return ceil_div(out_o, kNTile) * ceil_div(in_o, 32) * 32 * 64 * 16;
    return ceil_div(out_o, kNTile) * ceil_div(in_o, kKChunk) * 32 * 64 * (dtype == WALSH_BF16 ? 8 : 16);
}

WALSH_EXPORT int walsh_hadamard_dense_prepare(const float *w, int64_t in_o, int64_t out_o, int w_io, int dtype,
                                              uint8_t *kweight, void *stream) {
    const char *fn = "walsh_hadamard_dense_prepare";
    if (!w || !kweight) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (in_o <= 0 || out_o <= 0 || in_o > 65536 || out_o > 65536)
        return set_error(WALSH_EINVAL, "%s: bad shape in_o=%lld out_o=%lld", fn, (long long)in_o, (long long)out_o);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d", fn, dtype);
    const int Nt = (int)ceil_div(out_o, kNTile), Kc = (int)ceil_div(in_o, kKChunk);
    const int64_t total = (int64_t)Nt * Kc * 2048;
    int grid = (int)ceil_div(total, 256);
    if (grid > 4096) grid = 4096;
    if (dense_wide(in_o, out_o, dtype))
        launch(hadamard_dense_prepare32_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, w, (int)in_o,
               (int)out_o, w_io ? 1 : 0, Nt, (int)ceil_div(in_o, 32), (uint4 *)kweight);
    else
        launch(hadamard_dense_prepare_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, w, (int)in_o,
               (int)out_o, w_io ? 1 : 0, Nt, Kc, dtype == WALSH_BF16 ? 1 : 0, (unsigned char *)kweight);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_head_mixer_fwd(const void *x, int64_t B, int64_t T, int64_t D, int64_t x_bstride,
                                      int64_t x_hstride, int64_t x_tstride, const uint8_t *kweight,
                                      const float *beta, void *y, int64_t ldy, int dtype, void *stream) {
    const char *fn = "walsh_head_mixer_fwd";
    if (!x || !y || !kweight || !beta) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (B < 0 || T < 0 || D <= 0 || ldy < 32 * D || x_tstride < D || x_hstride < D)
        return set_error(WALSH_EINVAL, "%s: bad shape B=%lld T=%lld D=%lld", fn, (long long)B, (long long)T,
                         (long long)D);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d", fn, dtype);
    const bool wide = dense_wide(D, D, dtype);
    if (D > kDenseMaxO && !wide)
        return set_error(WALSH_ENOTSUP, "%s: head_dim %lld needs bf16 and <= %d (or <= %d)", fn, (long long)D,
                         kW3MaxO, kDenseMaxO);
    const int64_t M = B * T;
    if (M == 0) return WALSH_OK;
    const bool bf16 = dtype == WALSH_BF16;
    const int64_t esz = bf16 ? 2 : 4;
    // every offset of x and y stays inside a 31-bit buffer range
    const int64_t xspan = (B - 1) * x_bstride + 31 * x_hstride + (T - 1) * x_tstride + D;
    if (xspan * esz > (int64_t)kMaxBufferBytes || M * ldy * esz > (int64_t)kMaxBufferBytes || M > INT32_MAX)
        return set_error(WALSH_ENOTSUP, "%s: tensors above 2^31 bytes", fn);
    HadArgs a = had_args(x, x_tstride, x_hstride, D, D, kweight, nullptr, beta, y, ldy, D);
    a.kw3 = nullptr;
    a.beta_h = 0;  // one beta row for all heads
    a.M = (int)M;
    a.tpb = (int)T;
    a.bstride = x_bstride;
    a.xspan = xspan;
    if (wide) {
        if (D % 4 || x_hstride % 4 || x_tstride % 4 || x_bstride % 4 || ldy % 4 || (uintptr_t)x % 8 ||
            (uintptr_t)y % 8)
            return set_error(WALSH_ENOTSUP, "%s: head_dim %lld needs 4-aligned strides", fn, (long long)D);
        const size_t lds = wide3_lds_bytes((int)ceil_div(D, 32));
        if (lds > (size_t)device_info().max_shared_per_block)
            return set_error(WALSH_ENOTSUP, "%s: needs %zu B of LDS", fn, lds);
        if (M <= kSplitRows) {
            HadArgsN an;
            an.n = 1;
            an.p[0] = a;
            split3_launch(an, false, true, (hipStream_t)stream);
            return check_hip(hipGetLastError(), fn);
        }
        const int64_t items = ceil_div(M, kTile), cap = (int64_t)device_info().cu_count;
        launch(hadamard_wide3_kernel<0, true>, dim3((unsigned)(items < cap ? items : cap)), dim3(kWideThreads), lds,
               (hipStream_t)stream, a);
        return check_hip(hipGetLastError(), fn);
    }
    const int Nt = a.Nt, Kc = a.Kc;
    const size_t lds = (size_t)Nt * Kc * 32 * 64 * (bf16 ? 8 : 16) + (size_t)16 * 128 * (Kc + Nt);
    if (lds > (size_t)device_info().max_shared_per_block)
        return set_error(WALSH_ENOTSUP, "%s: head_dim %lld needs %zu B of LDS", fn, (long long)D, lds);
    const size_t valign = bf16 ? 8 : 16;
    const bool vec = D % 4 == 0 && x_hstride % 4 == 0 && x_tstride % 4 == 0 && x_bstride % 4 == 0 &&
                     (uintptr_t)x % valign == 0 && ldy % 4 == 0 && (uintptr_t)y % valign == 0;
    const bool kc1 = Kc == 1 && (bf16 || Nt == 1);
    if (bf16 && vec && kc1 && Nt == 1 && ceil_div(M, kTile) <= kPairMaxTiles) {
        // head_dim <= 16: a wavefront pair per tile
        HadArgsN an;
        an.n = 1;
        an.p[0] = a;
        pair_launch(an, M, (hipStream_t)stream, true);
        return check_hip(hipGetLastError(), fn);
    }
    int64_t grid = ceil_div(ceil_div(M, kTile), kWaves);
    const int64_t cap = (int64_t)device_info().cu_count * 2;
    if (grid > cap) grid = cap;
    const dim3 G((unsigned)grid), Bk(kThreads);
    hipStream_t s = (hipStream_t)stream;
#define WALSH_MIX_LAUNCH(T_, MMA, V, K1) launch((hadamard_fwd_kernel<T_, MMA, V, K1, true>), G, Bk, lds, s, a)
    if (bf16) {
        if (vec) { if (kc1) WALSH_MIX_LAUNCH(uint16_t, true, true, true); else WALSH_MIX_LAUNCH(uint16_t, true, true, false); }
        else     { if (kc1) WALSH_MIX_LAUNCH(uint16_t, true, false, true); else WALSH_MIX_LAUNCH(uint16_t, true, false, false); }
    } else {
        if (vec) { if (kc1) WALSH_MIX_LAUNCH(float, false, true, true); else WALSH_MIX_LAUNCH(float, false, true, false); }
        else     { if (kc1) WALSH_MIX_LAUNCH(float, false, false, true); else WALSH_MIX_LAUNCH(float, false, false, false); }
    }
#undef WALSH_MIX_LAUNCH
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_head_mixer_proj_fwd(const void *x, int64_t B, int64_t T, int64_t x_bstride, int64_t x_hstride,
                                           int64_t x_tstride, const uint8_t *mix_kweight, const float *mix_beta,
                                           const uint8_t *proj_kweight, const float *proj_alpha,
                                           const float *proj_beta, void *y, int64_t ldy, int dtype, void *stream) {
    const char *fn = "walsh_head_mixer_proj_fwd";
    if (!x || !y || !mix_kweight || !mix_beta || !proj_kweight || !proj_beta)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (B < 0 || T < 0 || ldy < 512 || x_tstride < 16 || x_hstride < 16 || x_bstride < 0)
        return set_error(WALSH_EINVAL, "%s: bad shape B=%lld T=%lld ldy=%lld", fn, (long long)B, (long long)T,
                         (long long)ldy);
    if (dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: bf16 only (dtype %d)", fn, dtype);
    if (x_hstride % 4 || x_tstride % 4 || x_bstride % 4 || ldy % 4 || (uintptr_t)x % 8 || (uintptr_t)y % 8)
        return set_error(WALSH_ENOTSUP, "%s: strides and pointers must be 4-element aligned", fn);
    const int64_t M = B * T;
    if (M == 0) return WALSH_OK;
    const int64_t xspan = (B - 1) * x_bstride + 31 * x_hstride + (T - 1) * x_tstride + 16;
    if (xspan * 2 > (int64_t)kMaxBufferBytes || M * ldy * 2 > (int64_t)kMaxBufferBytes || M > INT32_MAX)
        return set_error(WALSH_ENOTSUP, "%s: tensors above 2^31 bytes", fn);
    HadArgs m = had_args(x, x_tstride, x_hstride, 16, 16, mix_kweight, nullptr, mix_beta, y, ldy, 16);
    m.kw3 = nullptr;
    m.beta_h = 0;  // one beta row for all heads
    m.M = (int)M;
    m.tpb = (int)T;
    m.bstride = x_bstride;
    m.xspan = xspan;
    HadArgs p = had_args(y, ldy, 16, 16, 16, proj_kweight, proj_alpha, proj_beta, y, ldy, 16);
    p.M = (int)M;
    // one wavefront pair per 16-row tile, up to the pairs the CUs hold at
    // once (LDS: kMixProjLds each; registers: 2 wavefronts per SIMD, where
    // 3 would spill)
    int64_t per_cu = (int64_t)device_info().lds_per_cu / (int64_t)kMixProjLds;
    if (per_cu > 4) per_cu = 4;
    const int64_t resident = (int64_t)device_info().cu_count * per_cu;
    int64_t grid = ceil_div(M, kTile);
    if (grid > resident) grid = resident;
    launch(hadamard_pair_mixproj_kernel, dim3((unsigned)grid), dim3(kPairThreads), (uint32_t)kMixProjLds,
           (hipStream_t)stream, m, p);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_fht_fwd(const void *x, int64_t rows, int64_t n, int normalize, void *y, int dtype,
                               void *stream) {
    if (!x || !y) return set_error(WALSH_EINVAL, "walsh_fht_fwd: null pointer");
    if (rows < 0 || n < 1 || (n & (n - 1)) != 0 || n > 16384)
        return set_error(WALSH_EINVAL, "walsh_fht_fwd: n must be a power of two <= 16384 (got %lld)", (long long)n);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "walsh_fht_fwd: dtype");
    if (rows == 0) return WALSH_OK;
    int logN = 0;
    while ((1LL << logN) < n) ++logN;
    const int rpb = n >= 4096 ? 1 : (int)(4096 / n);
    const size_t lds = (size_t)rpb * n * 4;
    const float scale = normalize ? (float)(1.0 / sqrt((double)n)) : 1.0f;
    const dim3 G((unsigned)ceil_div(rows, rpb)), B(256);
    if (dtype == WALSH_BF16)
        launch(fht_kernel<uint16_t>, G, B, lds, (hipStream_t)stream, (const uint16_t *)x, rows, logN,
                           scale, (uint16_t *)y);
    else
        launch(fht_kernel<float>, G, B, lds, (hipStream_t)stream, (const float *)x, rows, logN, scale,
                           (float *)y);
    return check_hip(hipGetLastError(), "walsh_fht_fwd launch");
}
