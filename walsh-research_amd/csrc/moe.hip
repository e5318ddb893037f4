// Hadamard mixture-of-experts FFN (src/model/moe.py:306-560).
//
//   walsh_moe_route_fwd    HadamardRouter.forward (moe.py:418-447) fused:
//                          logits = W2 silu(W1 x); softmax; top-k (k =
//                          min(max_experts, E)); weights renormalised over
//                          the selected experts; per-expert token counts and
//                          probability sums (HadamardMoE._compute_aux_loss,
//                          moe.py:544-560); zero-fills the output blocks of
//                          unselected experts.
//   walsh_moe_topk_fwd     the same routing from given logits.
//   walsh_moe_scatter      per-expert token lists (exclusive scan of counts).
//   walsh_moe_experts_fwd  FastMoEExperts.forward (moe.py:337-380) on the
//                          selected (token, expert) pairs only: expert e maps
//                          the 32-wide block x[t, 32e:32e+32] through a ternary
//                          SwiGLU (gate/up [H, 32], down [32, H], codes times
//                          per-tensor gamma) and writes w * out into the same
//                          block of y.  Blocks are disjoint, so no atomics.
//
// Matrix-core layout.  Products are formed transposed (weights as the A
// operand, activations^T as B): the D fragment of one product -- lane
// (t = l % 16, q = l / 16) holding rows 4q..4q+3 of column t -- is exactly
// the B fragment the next product needs, so h1 feeds the logits and the
// expert hidden state feeds the down projection without a transpose.
#include <math.h>

#include "common.h"

namespace walsh {

constexpr int kMoeWaves = 4;
constexpr int kMoeThreads = 64 * kMoeWaves;
constexpr int kMaxETiles = 8;      // E <= 128
constexpr int kMaxK = 8;           // experts per token
constexpr int kHChunk = 8;         // router hidden tiles per pass (128 units)

// MMA step on a 16-wide K chunk whose 4-element slices sit in the lanes
// (A = 4 weights, B = 4 activations, as float4).
template <bool BF16MMA>
__device__ __forceinline__ f32x4 mma16(f32x4 a, f32x4 b, f32x4 acc) {
    if constexpr (BF16MMA) {
        uint2 av, bv;
        av.x = pack_bf16x2(a.x, a.y);
        av.y = pack_bf16x2(a.z, a.w);
        bv.x = pack_bf16x2(b.x, b.y);
        bv.y = pack_bf16x2(b.z, b.w);
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, av), __builtin_bit_cast(i16x4, bv),
                                                         acc, 0, 0, 0);
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
        return acc;
    }
}

__device__ __forceinline__ float silu_f(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// Round to the nearest bfloat16 and back: where the reference runs under
// bf16 autocast, every Linear/einsum output and elementwise result is a
// bf16 tensor, so the bf16 path rounds at the same points.
__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// ------------------------------------------------------------------ routing
struct RouteOut {
    int M, E, k;
    float *probs;     // [M, E] or null
    float *mask;      // [M, E] or null
    float *wdense;    // [M, E] or null
    int *topk_idx;    // [M, k]
    float *topk_w;    // [M, k]
    int *count;       // [E]  (accumulated)
    float *probsum;   // [E]  (accumulated)
    void *y;          // [M, ldy] or null: zero the blocks of unselected experts
    int64_t ldy;
    int y_bf16;
};

// Lane (t, q) of a 16-token tile holds lg[et][j] = logit of expert
// 16*et + 4q + j of token `tok`.  Softmax, top-k and outputs.
template <int NET>
__device__ __forceinline__ void route_tile(float (&lg)[NET][4], int net, int tok, bool tok_ok, int q,
                                           const RouteOut &o) {
    const int E = o.E;
    // softmax (fp32): max, exp, sum over the token's 4 lanes
    float mx = -INFINITY;
#pragma unroll
    for (int et = 0; et < NET; ++et)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 16 * et + 4 * q + j;
            if (et >= net || e >= E) lg[et][j] = -INFINITY;
            mx = fmaxf(mx, lg[et][j]);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float p[NET][4];
    float sum = 0.f;
#pragma unroll
    for (int et = 0; et < NET; ++et)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            p[et][j] = (lg[et][j] == -INFINITY) ? 0.f : expf(lg[et][j] - mx);
            sum += p[et][j];
        }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
#pragma unroll
    for (int et = 0; et < NET; ++et)
#pragma unroll
        for (int j = 0; j < 4; ++j) p[et][j] = __fdiv_rn(p[et][j], sum);

    // top-k: k rounds of (largest probability, lowest expert index on ties)
    unsigned sel[NET];  // bit j of sel[et]
#pragma unroll
    for (int et = 0; et < NET; ++et) sel[et] = 0;
    int idx_k[kMaxK];
    float p_k[kMaxK];
    float wsum = 0.f;
#pragma unroll
    for (int r = 0; r < kMaxK; ++r) {
        if (r >= o.k) break;
        float bv = -1.f;
        int be = 0x7fffffff;
#pragma unroll
        for (int et = 0; et < NET; ++et)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 16 * et + 4 * q + j;
                if (e < E && !((sel[et] >> j) & 1u) && (p[et][j] > bv || (p[et][j] == bv && e < be))) {
                    bv = p[et][j];
                    be = e;
                }
            }
#pragma unroll
        for (int sh = 16; sh <= 32; sh <<= 1) {
            const float ov = __shfl_xor(bv, sh);
            const int oe = __shfl_xor(be, sh);
            if (ov > bv || (ov == bv && oe < be)) {
                bv = ov;
                be = oe;
            }
        }
        // the owner lane marks it
        const int wet = be >> 4, wq = (be >> 2) & 3, wj = be & 3;
#pragma unroll
        for (int et = 0; et < NET; ++et)
            if (et == wet && wq == q) sel[et] |= 1u << wj;
        idx_k[r] = be;
        p_k[r] = bv;
        wsum += bv;
    }
    const float den = fmaxf(wsum, 1e-8f);
    if (tok_ok && q == 0) {
#pragma unroll
        for (int r = 0; r < kMaxK; ++r) {
            if (r >= o.k) break;
            o.topk_idx[(int64_t)tok * o.k + r] = idx_k[r];
            o.topk_w[(int64_t)tok * o.k + r] = __fdiv_rn(p_k[r], den);
        }
    }
    // dense outputs and zero blocks for the unselected experts of this lane
#pragma unroll
    for (int et = 0; et < NET; ++et) {
        if (et >= net) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 16 * et + 4 * q + j;
            if (!tok_ok || e >= E) continue;
            const bool s = (sel[et] >> j) & 1u;
            const int64_t pe = (int64_t)tok * E + e;
            if (o.probs) o.probs[pe] = p[et][j];
            if (o.mask) o.mask[pe] = s ? 1.f : 0.f;
            if (o.wdense) o.wdense[pe] = s ? __fdiv_rn(p[et][j], den) : 0.f;
            if (o.y && !s) {
                if (o.y_bf16) {
                    uint4 *d = (uint4 *)((uint16_t *)o.y + tok * o.ldy + 32 * e);
#pragma unroll
                    for (int z = 0; z < 4; ++z) d[z] = uint4{0, 0, 0, 0};
                } else {
                    uint4 *d = (uint4 *)((float *)o.y + tok * o.ldy + 32 * e);
#pragma unroll
                    for (int z = 0; z < 8; ++z) d[z] = uint4{0, 0, 0, 0};
                }
            }
        }
    }
    // per-expert count and probability sum over the tile's 16 tokens
#pragma unroll
    for (int et = 0; et < NET; ++et) {
        if (et >= net) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float c = (tok_ok && ((sel[et] >> j) & 1u)) ? 1.f : 0.f;
            float ps = tok_ok ? p[et][j] : 0.f;
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) {
                c += __shfl_xor(c, sh);
                ps += __shfl_xor(ps, sh);
            }
            const int e = 16 * et + 4 * q + j;
            if ((threadIdx.x & 15) == 0 && e < E) {
                if (c > 0.f) atomicAdd(o.count + e, (int)c);
                atomicAdd(o.probsum + e, ps);
            }
        }
    }
}

struct RouterArgs {
    const void *x;
    int64_t ldx;
    int C, H1;
    const void *w1f;   // [H1/16][C/16][64][4]   W1[16nt+m][16ks+4kq+j]
    const void *w2f;   // [ET][H1/16][64][4]     W2[16et+m][16ks+4kq+j]
    int net;
    RouteOut o;
};

template <typename T, bool BF16MMA, int NET>
__global__ __launch_bounds__(kMoeThreads, 2) void moe_route_kernel(RouterArgs a) {
    constexpr uint32_t esz = sizeof(T);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = lane & 15, q = lane >> 4;
    const int M = a.o.M;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)M * a.ldx * esz));
    const int nks = a.C / 16, nht = a.H1 / 16;
    const __amdgpu_buffer_rsrc_t w1r = make_rsrc(a.w1f, (uint32_t)((int64_t)nht * nks * 256 * esz));
    const __amdgpu_buffer_rsrc_t w2r = make_rsrc(a.w2f, (uint32_t)((int64_t)a.net * nht * 256 * esz));
    const int n_tiles = (int)ceil_div(M, 16);
    for (int tile = blockIdx.x * kMoeWaves + wave; tile < n_tiles; tile += gridDim.x * kMoeWaves) {
        const int tok = tile * 16 + t;
        const bool tok_ok = tok < M;
        const uint32_t xo = tok_ok ? (uint32_t)((int64_t)tok * a.ldx * esz) : kOOB;
        f32x4 lg[NET];
#pragma unroll
        for (int et = 0; et < NET; ++et) lg[et] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int hc = 0; hc < nht; hc += kHChunk) {
            f32x4 h[kHChunk];
#pragma unroll
            for (int i = 0; i < kHChunk; ++i) h[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            for (int ks = 0; ks < nks; ++ks) {
                const f32x4 xb = Buf4<T>::load(xr, xo == kOOB ? kOOB : xo + (uint32_t)(16 * ks + 4 * q) * esz, 0);
#pragma unroll
                for (int i = 0; i < kHChunk; ++i) {
                    const int nt = hc + i;
                    const f32x4 w = Buf4<T>::load(
                        w1r, nt < nht ? (uint32_t)((((int64_t)nt * nks + ks) * 64 + lane) * 4 * esz) : kOOB, 0);
                    h[i] = mma16<BF16MMA>(w, xb, h[i]);
                }
            }
            // h1 = silu(.) (rounded to the operand type), then logits += W2[:, chunk] h1
#pragma unroll
            for (int i = 0; i < kHChunk; ++i) {
                const int nt = hc + i;
                if (nt >= nht) break;
                f32x4 hb;
#pragma unroll
                for (int j = 0; j < 4; ++j) hb[j] = BF16MMA ? bf16r(silu_f(bf16r(h[i][j]))) : silu_f(h[i][j]);
#pragma unroll
                for (int et = 0; et < NET; ++et) {
                    if (et >= a.net) break;
                    const f32x4 w = Buf4<T>::load(w2r, (uint32_t)((((int64_t)et * nht + nt) * 64 + lane) * 4 * esz), 0);
                    lg[et] = mma16<BF16MMA>(w, hb, lg[et]);
                }
            }
        }
        float l2[NET][4];
#pragma unroll
        for (int et = 0; et < NET; ++et)
#pragma unroll
            for (int j = 0; j < 4; ++j) l2[et][j] = BF16MMA ? bf16r(lg[et][j]) : lg[et][j];
        route_tile(l2, a.net, tok, tok_ok, q, a.o);
    }
}

template <int NET>
__global__ __launch_bounds__(kMoeThreads) void moe_topk_kernel(const float *__restrict__ logits, int net,
                                                               RouteOut o) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = lane & 15, q = lane >> 4;
    const int n_tiles = (int)ceil_div(o.M, 16);
    for (int tile = blockIdx.x * kMoeWaves + wave; tile < n_tiles; tile += gridDim.x * kMoeWaves) {
        const int tok = tile * 16 + t;
        const bool tok_ok = tok < o.M;
        float lg[NET][4];
#pragma unroll
        for (int et = 0; et < NET; ++et)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 16 * et + 4 * q + j;
                lg[et][j] = (tok_ok && et < net && e < o.E) ? logits[(int64_t)tok * o.E + e] : -INFINITY;
            }
        route_tile(lg, net, tok, tok_ok, q, o);
    }
}

__global__ void moe_zero_kernel(int *count, float *probsum, int *cursor, int E) {
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        count[e] = 0;
        probsum[e] = 0.f;
        cursor[e] = 0;
    }
}

// ------------------------------------------------------------------ scatter
// Every block scans the E counts itself (E <= 128), then places its pairs:
// list[offset[e] + atomic cursor[e]] = pair id (t*k + j).  Block 0 also
// publishes offset[E+1] and tile_off[E+1] (16-pair tiles per expert).
__global__ __launch_bounds__(256) void moe_scatter_kernel(const int *__restrict__ topk_idx, int64_t n_pairs, int E,
                                                          const int *__restrict__ count, int *__restrict__ cursor,
                                                          int *__restrict__ list, int *__restrict__ offset,
                                                          int *__restrict__ tile_off) {
    __shared__ int off_s[129];
    if (threadIdx.x == 0) {
        int acc = 0, tacc = 0;
        for (int e = 0; e < E; ++e) {
            off_s[e] = acc;
            if (blockIdx.x == 0) {
                offset[e] = acc;
                tile_off[e] = tacc;
            }
            acc += count[e];
            tacc += (count[e] + 15) / 16;
        }
        off_s[E] = acc;
        if (blockIdx.x == 0) {
            offset[E] = acc;
            tile_off[E] = tacc;
        }
    }
    __syncthreads();
    for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < n_pairs; p += (int64_t)gridDim.x * blockDim.x) {
        const int e = topk_idx[p];
        const int pos = off_s[e] + atomicAdd(cursor + e, 1);
        list[pos] = (int)p;
    }
}

// ------------------------------------------------------------------ experts
struct ExpArgs {
    const void *x;
    int64_t ldx;
    void *y;
    int64_t ldy;
    int M, E, k, H;                // H = hidden units per expert (multiple of 16)
    const uint8_t *gate_f;         // [E][H/16][2][64]  packed codes, A fragments
    const uint8_t *up_f;           // [E][H/16][2][64]
    const uint8_t *down_f;         // [E][2][H/16][64]
    const float *gammas;           // gate, up, down
    const int *list, *offset, *tile_off, *count;
    const float *topk_w;           // [M*k]
};

template <typename T, typename TY, bool BF16MMA, int NHT>
__global__ __launch_bounds__(kMoeThreads, 2) void moe_experts_kernel(ExpArgs a) {
    __shared__ __align__(16) f32x4 lut[256];
    __shared__ int toff[129];
    {
        const uint32_t byte = threadIdx.x;
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (float)((int)((byte >> (6 - 2 * j)) & 3u) - 1);
        lut[byte] = v;
    }
    for (int e = threadIdx.x; e <= a.E; e += kMoeThreads) toff[e] = a.tile_off[e];
    __syncthreads();
    constexpr uint32_t esz = sizeof(T);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = lane & 15, q = lane >> 4;
    constexpr int nht = NHT;                  // hidden tiles of 16 (H = 16 * NHT)
    const float gg = a.gammas[0], gu = a.gammas[1], gd = a.gammas[2];
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * esz));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)((int64_t)a.M * a.ldy * sizeof(TY)));
    const int total = toff[a.E];
    for (int item = blockIdx.x * kMoeWaves + wave; item < total; item += gridDim.x * kMoeWaves) {
        int lo = 0, hi = a.E - 1;  // expert with toff[e] <= item < toff[e+1]
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (toff[mid] <= item) lo = mid; else hi = mid - 1;
        }
        const int e = lo;
        const int local = item - toff[e];
        const int cnt = min(16, a.count[e] - 16 * local);
        const bool ok = t < cnt;
        const int pair = ok ? a.list[a.offset[e] + 16 * local + t] : 0;
        const int tok = pair / a.k;
        const float wr = ok ? a.topk_w[pair] : 0.f;
        const uint32_t xo = ok ? (uint32_t)(((int64_t)tok * a.ldx + 32 * e) * esz) : kOOB;
        f32x4 xb[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) xb[c] = Buf4<T>::load(xr, xo == kOOB ? kOOB : xo + (uint32_t)(16 * c + 4 * q) * esz, 0);
        // gate/up: D[hidden][pair]; lane (t, q) ends with hidden 16nt + 4q + j of pair t
        f32x4 hb[NHT];
        const uint8_t *gf = a.gate_f + (int64_t)e * nht * 128;
        const uint8_t *uf = a.up_f + (int64_t)e * nht * 128;
#pragma unroll
        for (int nt = 0; nt < nht; ++nt) {
            f32x4 g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                g = mma16<BF16MMA>(lut[gf[(nt * 2 + c) * 64 + lane]], xb[c], g);
                u = mma16<BF16MMA>(lut[uf[(nt * 2 + c) * 64 + lane]], xb[c], u);
            }
            f32x4 h;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (BF16MMA) {
                    h[j] = bf16r(silu_f(bf16r(gg * g[j]))) * bf16r(gu * u[j]);
                } else {
                    h[j] = silu_f(gg * g[j]) * (gu * u[j]);
                }
            }
            hb[nt] = h;
        }
        // down: D[d][pair], 2 tiles of 16 output dims, K = H in steps of 16
        const uint8_t *df = a.down_f + (int64_t)e * nht * 128;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < nht; ++ks) d = mma16<BF16MMA>(lut[df[(mt * nht + ks) * 64 + lane]], hb[ks], d);
            f32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = (BF16MMA ? bf16r(gd * d[j]) : gd * d[j]) * wr;
            Buf4<TY>::store(o, yr,
                            xo == kOOB ? kOOB
                                       : (uint32_t)(((int64_t)tok * a.ldy + 32 * e + 16 * mt + 4 * q) * sizeof(TY)),
                            0);
        }
    }
}

}  // namespace walsh

using namespace walsh;

static int grid_cap(int64_t waves_needed) {
    int64_t g = ceil_div(waves_needed, kMoeWaves);
    const int64_t cap = (int64_t)device_info().cu_count * 4;
    if (g > cap) g = cap;
    return (int)(g < 1 ? 1 : g);
}

static int route_out_check(const char *fn, int64_t M, int64_t E, int64_t k, const int *topk_idx, const float *topk_w,
                           const int *count, const float *probsum) {
    if (!count || !probsum || (M > 0 && (!topk_idx || !topk_w)))
        return set_error(WALSH_EINVAL, "%s: null output pointer", fn);
    if (M < 0 || E < 1 || E > 16 * kMaxETiles || k < 1 || k > kMaxK || k > E)
        return set_error(WALSH_ENOTSUP, "%s: needs 1 <= k <= min(E, %d) and E <= %d (M=%lld E=%lld k=%lld)", fn, kMaxK,
                         16 * kMaxETiles, (long long)M, (long long)E, (long long)k);
    return WALSH_OK;
}

WALSH_EXPORT int walsh_moe_route_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, int64_t H1, const void *w1_frag,
                                     const void *w2_frag, int64_t E, int64_t k, float *probs, float *mask,
                                     float *weights_dense, int *topk_idx, float *topk_w, int *count, float *probsum,
                                     int *cursor, void *y, int64_t ldy, int dtype, int ydtype, void *stream) {
    const char *fn = "walsh_moe_route_fwd";
    int rc = route_out_check(fn, M, E, k, topk_idx, topk_w, count, probsum);
    if (rc) return rc;
    if ((M > 0 && !x) || !w1_frag || !w2_frag || !cursor) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (C % 16 || H1 % 16 || C < 16 || H1 < 16 || ldx < C || (y && ldy < 32 * E))
        return set_error(WALSH_ENOTSUP, "%s: needs C %% 16 == 0 and H1 %% 16 == 0 (C=%lld H1=%lld)", fn, (long long)C,
                         (long long)H1);
    if (E > 64) return set_error(WALSH_ENOTSUP, "%s: fused router needs E <= 64 (use walsh_moe_topk_fwd)", fn);
    if ((dtype != WALSH_F32 && dtype != WALSH_BF16) || (ydtype != WALSH_F32 && ydtype != WALSH_BF16))
        return set_error(WALSH_ENOTSUP, "%s: dtype", fn);
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4, ysz = ydtype == WALSH_BF16 ? 2 : 4;
    if (ldx % (16 / esz) || (uintptr_t)x % 16 || (y && ((uintptr_t)y % 16 || ldy % (16 / ysz))))
        return set_error(WALSH_ENOTSUP, "%s: x and y rows must be 16-byte aligned", fn);
    if (M * ldx * esz > (int64_t)kMaxBufferBytes) return set_error(WALSH_ENOTSUP, "%s: input too large", fn);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(moe_zero_kernel, dim3(1), dim3(128), 0, s, count, probsum, cursor, (int)E);
    if (M == 0) return check_hip(hipGetLastError(), fn);
    RouterArgs a;
    a.x = x;
    a.ldx = ldx;
    a.C = (int)C;
    a.H1 = (int)H1;
    a.w1f = w1_frag;
    a.w2f = w2_frag;
    a.net = (int)ceil_div(E, 16);
    a.o = RouteOut{(int)M, (int)E, (int)k, probs, mask, weights_dense, topk_idx, topk_w, count, probsum, y, ldy,
                   ydtype == WALSH_BF16};
    const dim3 G(grid_cap(ceil_div(M, 16))), B(kMoeThreads);
#define WALSH_ROUTE(NE)                                                                               \
    if (dtype == WALSH_BF16) hipLaunchKernelGGL((moe_route_kernel<uint16_t, true, NE>), G, B, 0, s, a); \
    else hipLaunchKernelGGL((moe_route_kernel<float, false, NE>), G, B, 0, s, a);
    if (a.net <= 1) { WALSH_ROUTE(1) } else if (a.net <= 2) { WALSH_ROUTE(2) } else { WALSH_ROUTE(4) }
#undef WALSH_ROUTE
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_moe_topk_fwd(const float *logits, int64_t M, int64_t E, int64_t k, float *probs, float *mask,
                                    float *weights_dense, int *topk_idx, float *topk_w, int *count, float *probsum,
                                    int *cursor, void *stream) {
    const char *fn = "walsh_moe_topk_fwd";
    int rc = route_out_check(fn, M, E, k, topk_idx, topk_w, count, probsum);
    if (rc) return rc;
    if ((M > 0 && !logits) || !cursor) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(moe_zero_kernel, dim3(1), dim3(128), 0, s, count, probsum, cursor, (int)E);
    if (M == 0) return check_hip(hipGetLastError(), fn);
    RouteOut o{(int)M, (int)E, (int)k, probs, mask, weights_dense, topk_idx, topk_w, count, probsum, nullptr, 0, 0};
    const int net = (int)ceil_div(E, 16);
    const dim3 G(grid_cap(ceil_div(M, 16))), B(kMoeThreads);
    if (net <= 1) hipLaunchKernelGGL(moe_topk_kernel<1>, G, B, 0, s, logits, net, o);
    else if (net <= 2) hipLaunchKernelGGL(moe_topk_kernel<2>, G, B, 0, s, logits, net, o);
    else if (net <= 4) hipLaunchKernelGGL(moe_topk_kernel<4>, G, B, 0, s, logits, net, o);
    else hipLaunchKernelGGL(moe_topk_kernel<8>, G, B, 0, s, logits, net, o);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_moe_scatter(const int *topk_idx, int64_t M, int64_t E, int64_t k, const int *count, int *cursor,
                                   int *list, int *offset, int *tile_off, void *stream) {
    if ((M > 0 && (!topk_idx || !list)) || !count || !cursor || !offset || !tile_off)
        return set_error(WALSH_EINVAL, "walsh_moe_scatter: null pointer");
    if (M < 0 || E < 1 || E > 128 || k < 1) return set_error(WALSH_EINVAL, "walsh_moe_scatter: bad shape");
    const int64_t n_pairs = M * k;
    int64_t grid = ceil_div(n_pairs, 256);
    if (grid > (int64_t)device_info().cu_count * 4) grid = (int64_t)device_info().cu_count * 4;
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL(moe_scatter_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, topk_idx, n_pairs,
                       (int)E, count, cursor, list, offset, tile_off);
    return check_hip(hipGetLastError(), "walsh_moe_scatter launch");
}

WALSH_EXPORT int walsh_moe_experts_fwd(const void *x, int64_t ldx, void *y, int64_t ldy, int64_t M, int64_t E,
                                       int64_t k, int64_t H, const uint8_t *gate_frag, const uint8_t *up_frag,
                                       const uint8_t *down_frag, const float *gammas, const int *list,
                                       const int *offset, const int *tile_off, const int *count,
                                       const float *topk_w, int dtype, int ydtype, void *stream) {
    const char *fn = "walsh_moe_experts_fwd";
    if (!x || !y || !gate_frag || !up_frag || !down_frag || !gammas || !list || !offset || !tile_off || !count ||
        !topk_w)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || E < 1 || E > 128 || k < 1 || (H != 64 && H != 128 && H != 256) || ldx < 32 * E || ldy < 32 * E)
        return set_error(WALSH_ENOTSUP, "%s: needs E <= 128 and hidden H in {64, 128, 256} (expansion 2/4/8)", fn);
    if (!((dtype == WALSH_F32 && ydtype == WALSH_F32) || (dtype == WALSH_BF16 && ydtype == WALSH_BF16) ||
          (dtype == WALSH_BF16 && ydtype == WALSH_F32)))
        return set_error(WALSH_ENOTSUP, "%s: (dtype, ydtype) must be (f32, f32), (bf16, bf16) or (bf16, f32)", fn);
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4, ysz = ydtype == WALSH_BF16 ? 2 : 4;
    if (ldx % (16 / esz) || ldy % (16 / ysz) || (uintptr_t)x % 16 || (uintptr_t)y % 16)
        return set_error(WALSH_ENOTSUP, "%s: x and y rows must be 16-byte aligned", fn);
    if (M * ldx * esz > (int64_t)kMaxBufferBytes || M * ldy * ysz > (int64_t)kMaxBufferBytes)
        return set_error(WALSH_ENOTSUP, "%s: input too large", fn);
    if (M == 0) return WALSH_OK;
    ExpArgs a;
    a.x = x;
    a.ldx = ldx;
    a.y = y;
    a.ldy = ldy;
    a.M = (int)M;
    a.E = (int)E;
    a.k = (int)k;
    a.H = (int)H;
    a.gate_f = gate_frag;
    a.up_f = up_frag;
    a.down_f = down_frag;
    a.gammas = gammas;
    a.list = list;
    a.offset = offset;
    a.tile_off = tile_off;
    a.count = count;
    a.topk_w = topk_w;
    // upper bound on 16-pair tiles: ceil(M*k/16) + E
    const dim3 G(grid_cap(ceil_div(M * k, 16) + E)), B(kMoeThreads);
    hipStream_t s = (hipStream_t)stream;
#define WALSH_EXP_LAUNCH(NH)                                                                                  \
    if (dtype == WALSH_F32) hipLaunchKernelGGL((moe_experts_kernel<float, float, false, NH>), G, B, 0, s, a);  \
    else if (ydtype == WALSH_BF16)                                                                            \
        hipLaunchKernelGGL((moe_experts_kernel<uint16_t, uint16_t, true, NH>), G, B, 0, s, a);                \
    else hipLaunchKernelGGL((moe_experts_kernel<uint16_t, float, true, NH>), G, B, 0, s, a);
    if (H == 64) { WALSH_EXP_LAUNCH(4) } else if (H == 128) { WALSH_EXP_LAUNCH(8) } else { WALSH_EXP_LAUNCH(16) }
#undef WALSH_EXP_LAUNCH
    return check_hip(hipGetLastError(), fn);
}
