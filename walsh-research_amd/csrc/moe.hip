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
#include "gemm256.h"

namespace walsh {

constexpr int kMoeWaves = 4;
constexpr int kMoeThreads = 64 * kMoeWaves;
constexpr int kMaxETiles = 8;      // E <= 128
constexpr int kMaxE = 16 * kMaxETiles;
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


// ------------------------------------------------------------------ routing
struct RouteOut {
    int M, E, k;
    float *probs;     // [M, E] or null
    float *mask;      // [M, E] or null
    float *wdense;    // [M, E] or null
    int *topk_idx;    // [M, k]
    float *topk_w;    // [M, k]
    int *count;       // [n_part][E] per-workgroup partial sums
    float *probsum;   // [n_part][E]
    int n_part;
    void *y;          // [M, ldy] or null: zero the blocks of unselected experts
    int64_t ldy;
    int y_bf16;
};

// Softmax and top-k of one 16-token tile.  Lane (t, q) holds lg[et][j] =
// logit of expert 16*et + 4q + j of its token; the token's 4 lanes (q = 0..3)
// cooperate through cross-lane exchanges: the lanes of quads q ^ 1 and q ^ 2
// are lane ^ X1 and lane ^ X2 (16 and 32 for t = lane % 16, q = lane / 16;
// 1 and 2 for q = lane % 4, whose exchanges stay inside a DPP quad).  Results: p = probabilities,
// rank = position of each of the lane's experts in the token's order
// (largest probability first, lower expert index on ties; >= k when not
// selected), sel = bit j of sel[et] set when rank[et][j] < k, and den =
// max(sum of the selected probabilities, 1e-8).
template <int NET> struct TopK {
    float p[NET][4];
    int rank[NET][4];
    unsigned sel[NET];
    float den;
};

// The value of lane (l ^ X): X = 16 or 32 through ds_bpermute; X = 1 or 2
// (lanes of one quad) as a DPP quad permutation, a modifier on a VALU move
// with no LDS round trip.
template <int X> __device__ __forceinline__ int xchg_i(int v) {
    if constexpr (X == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
    else if constexpr (X == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    else return __shfl_xor(v, X);
}
template <int X> __device__ __forceinline__ float xchg(float v) { return __int_as_float(xchg_i<X>(__float_as_int(v))); }

// The value of lane l - N of the same 16-lane row (DPP row_shr; 0 where
// l - N falls before the row).
template <int N> __device__ __forceinline__ float row_shr(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + N, 0xf, 0xf, true));
}

// x > y in the routing order (ties: the lower expert index wins; lower_x
// says whether x's expert index is the lower one).
__device__ __forceinline__ int beats(float x, float y, bool lower_x) { return (x > y) || (x == y && lower_x); }

template <int NET, int X1 = 16, int X2 = 32>
__device__ __forceinline__ void topk_core(float (&lg)[NET][4], int net, int E, int k, int q, TopK<NET> &r) {
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
    mx = fmaxf(mx, xchg<X1>(mx));
    mx = fmaxf(mx, xchg<X2>(mx));
    float sum = 0.f;
#pragma unroll
    for (int et = 0; et < NET; ++et)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r.p[et][j] = (lg[et][j] == -INFINITY) ? 0.f : expf(lg[et][j] - mx);
            sum += r.p[et][j];
        }
    sum += xchg<X1>(sum);
    sum += xchg<X2>(sum);
#pragma unroll
    for (int et = 0; et < NET; ++et)
#pragma unroll
        for (int j = 0; j < 4; ++j) r.p[et][j] = __fdiv_rn(r.p[et][j], sum);

    if constexpr (NET == 1) {
        // E <= 16: every lane of the token gathers all 16 probabilities and
        // ranks its own 4 by counting the entries that beat them.
        float o[4], a1[4], a2[4], a3[4];  // experts 4q+j, 4(q^1)+j, 4(q^2)+j, 4(q^3)+j
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = (4 * q + j < E) ? r.p[0][j] : -1.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a1[j] = xchg<X1>(o[j]);
            a2[j] = xchg<X2>(o[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) a3[j] = xchg<X2>(a1[j]);
        const bool l1 = (q ^ 1) < q, l2 = (q ^ 2) < q, l3 = (q ^ 3) < q;
        float ssum = 0.f;
        r.sel[0] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int rk = 0;
#pragma unroll
            for (int j2 = 0; j2 < 4; ++j2) {
                if (j2 != j) rk += beats(o[j2], o[j], j2 < j);
                rk += beats(a1[j2], o[j], l1);
                rk += beats(a2[j2], o[j], l2);
                rk += beats(a3[j2], o[j], l3);
            }
            const bool s = rk < k && 4 * q + j < E;
            r.rank[0][j] = s ? rk : kMaxE;
            r.sel[0] |= s ? 1u << j : 0u;
            ssum += s ? r.p[0][j] : 0.f;
        }
        ssum += xchg<X1>(ssum);
        ssum += xchg<X2>(ssum);
        r.den = fmaxf(ssum, 1e-8f);
    } else {
        // k rounds of (largest probability, lowest expert index on ties)
#pragma unroll
        for (int et = 0; et < NET; ++et) {
            r.sel[et] = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) r.rank[et][j] = kMaxE;
        }
        float wsum = 0.f;
#pragma unroll
        for (int i = 0; i < kMaxK; ++i) {
            if (i >= k) break;
            float bv = -1.f;
            int be = 0x7fffffff;
#pragma unroll
            for (int et = 0; et < NET; ++et)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int e = 16 * et + 4 * q + j;
                    const bool better = e < E && !((r.sel[et] >> j) & 1u) && beats(r.p[et][j], bv, e < be);
                    bv = better ? r.p[et][j] : bv;
                    be = better ? e : be;
                }
            {
                const float ov = xchg<X1>(bv);
                const int oe = xchg_i<X1>(be);
                const bool better = beats(ov, bv, oe < be);
                bv = better ? ov : bv;
                be = better ? oe : be;
            }
            {
                const float ov = xchg<X2>(bv);
                const int oe = xchg_i<X2>(be);
                const bool better = beats(ov, bv, oe < be);
                bv = better ? ov : bv;
                be = better ? oe : be;
            }
            // the owner lane marks it
            const int wet = be >> 4, wq = (be >> 2) & 3, wj = be & 3;
#pragma unroll
            for (int et = 0; et < NET; ++et)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (et == wet && wq == q && j == wj) {
                        r.sel[et] |= 1u << j;
                        r.rank[et][j] = i;
                    }
            wsum += bv;
        }
        r.den = fmaxf(wsum, 1e-8f);
    }
}

// Zero the 32-element output block starting at element `at` of y.
__device__ __forceinline__ void zero_block(void *y, int bf16, int64_t at) {
    if (bf16) {
        uint4 *d = (uint4 *)((uint16_t *)y + at);
#pragma unroll
        for (int z = 0; z < 4; ++z) d[z] = uint4{0, 0, 0, 0};
    } else {
        uint4 *d = (uint4 *)((float *)y + at);
#pragma unroll
        for (int z = 0; z < 8; ++z) d[z] = uint4{0, 0, 0, 0};
    }
}

// Outputs of a routed tile (see RouteOut); counts go to the workgroup's LDS
// counters cnt_l, probability sums to this wave's row ps_w (PartSums).
template <int NET>
__device__ __forceinline__ void route_tile(float (&lg)[NET][4], int net, int tok, bool tok_ok, int q,
                                           const RouteOut &o, int *cnt_l, float *ps_w) {
    const int E = o.E;
    TopK<NET> r;
    topk_core<NET>(lg, net, E, o.k, q, r);
    const float den = r.den;
    float (&p)[NET][4] = r.p;
    unsigned (&sel)[NET] = r.sel;
    // each lane writes the top-k entries of its own selected experts
#pragma unroll
    for (int et = 0; et < NET; ++et)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (tok_ok && ((sel[et] >> j) & 1u)) {
                const int64_t at = (int64_t)tok * o.k + r.rank[et][j];
                o.topk_idx[at] = 16 * et + 4 * q + j;
                o.topk_w[at] = __fdiv_rn(p[et][j], den);
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
            if (o.y && !s) zero_block(o.y, o.y_bf16, tok * o.ldy + 32 * e);
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
                if (c > 0.f) atomicAdd(cnt_l + e, (int)c);
                ps_w[e] += ps;
            }
        }
    }
}

// Per-workgroup partial sums in LDS.  Counts: integer atomics (exact in any
// order).  Probability sums: one row per wave, each row written only by its
// own wave (the lanes of one instruction add to distinct experts) and the
// rows added in wave order by part_store, so the float sums are the same on
// every run.
constexpr int kPartRows = 8;
struct PartSums {
    int cnt[kMaxE];
    float ps[kPartRows][kMaxE];
};

__device__ __forceinline__ void part_init(PartSums &s) {
    for (int i = threadIdx.x; i < kPartRows * kMaxE; i += blockDim.x) {
        s.ps[i / kMaxE][i % kMaxE] = 0.f;
        if (i < kMaxE) s.cnt[i] = 0;
    }
}

// Store this workgroup's partial sums in row blockIdx.x (and zero the rows
// no workgroup of this launch owns).  Same-address global atomics from
// every workgroup would serialise across the chip.
__device__ __forceinline__ void part_store(const PartSums &s, int *count, float *probsum, int E, int n_part) {
    __syncthreads();
    const int rows = (int)(blockDim.x >> 6) < kPartRows ? (int)(blockDim.x >> 6) : kPartRows;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        float ps = s.ps[0][e];
        for (int w = 1; w < rows; ++w) ps += s.ps[w][e];
        count[(int64_t)blockIdx.x * E + e] = s.cnt[e];
        probsum[(int64_t)blockIdx.x * E + e] = ps;
        for (int r = blockIdx.x + gridDim.x; r < n_part; r += gridDim.x) {
            count[(int64_t)r * E + e] = 0;
            probsum[(int64_t)r * E + e] = 0.f;
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
    __shared__ PartSums part;
    part_init(part);
    __syncthreads();
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
        route_tile(l2, a.net, tok, tok_ok, q, a.o, part.cnt, part.ps[wave]);
    }
    part_store(part, a.o.count, a.o.probsum, a.o.E, a.o.n_part);
}

template <int NET>
__global__ __launch_bounds__(kMoeThreads) void moe_topk_kernel(const float *__restrict__ logits, int net,
                                                               RouteOut o) {
    __shared__ PartSums part;
    part_init(part);
    __syncthreads();
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
        route_tile(lg, net, tok, tok_ok, q, o, part.cnt, part.ps[wave]);
    }
    part_store(part, o.count, o.probsum, o.E, o.n_part);
}

// Top-k routing for 16 < E <= 128 experts: one wavefront per token, lane l
// holding experts l and l + 64.  Softmax by wave reductions (max, then a
// fixed-order sum); the k selected experts come from k rounds of a wave
// argmax (largest probability, ties to the lower expert index), each round a
// register max over the wave and a ballot of the lanes holding it, so no LDS
// round trip and O(k) instead of O(E) steps per lane.  Same outputs as
// moe_topk_kernel.
//
// Wave reductions on the VALU: DPP moves within each row of 16 lanes and the
// gfx950 permlane16/32 swaps across rows (with both operands equal a swap
// returns a lane's value and its partner's, lanes i ^ 16 or i ^ 32).
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]: lanes ^ 1
    v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]: lanes ^ 2
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror: the other quad of 8
    v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror: the other 8 of the row
    const u32x2v a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a.x), __uint_as_float(a.y));
    const u32x2v b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b.x), __uint_as_float(b.y));
}
// Sum over the wave as the butterfly v += v[lane ^ s] for s = 32, 16, 8, 4,
// 2, 1 (every lane ends with the same, order-fixed value).  Within a row the
// partner comes from a rotation by s: after the steps of 2s, 4s, .. the row's
// values depend only on lane mod 2s, where lane + s and lane ^ s agree.
__device__ __forceinline__ float wave_sum(float v) {
    const u32x2v b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(b.x) + __uint_as_float(b.y);
    const u32x2v a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a.x) + __uint_as_float(a.y);
    v += dpp_f<0x128>(v);  // row_ror 8
    v += dpp_f<0x124>(v);  // row_ror 4
    v += dpp_f<0x122>(v);  // row_ror 2
    v += dpp_f<0x121>(v);  // row_ror 1
    return v;
}

// Softmax, top-k and the routing outputs of token `tok`, whose logits the
// wave holds as lg[0] (expert lane) and lg[1] (expert lane + 64), -inf past
// E.  Every lane of the wave takes part.
__device__ __forceinline__ void rank_token(int tok, const float (&lg)[2], const RouteOut &o, int *cnt_l,
                                           float *ps_w, int *sel_l = nullptr) {
    const int lane = threadIdx.x & 63;
    const int E = o.E, k = o.k;
    float p[2];
    int e[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) e[h] = lane + 64 * h;
    const float mx = wave_max(fmaxf(lg[0], lg[1]));
#pragma unroll
    for (int h = 0; h < 2; ++h) p[h] = (lg[h] == -INFINITY) ? 0.f : expf(lg[h] - mx);
    const float sum = wave_sum(p[0] + p[1]);
    // q: the candidates of the argmax rounds; probabilities are >= 0, entries
    // past E hold -1 and a selected entry -inf, so neither wins again
    float q[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        p[h] = __fdiv_rn(p[h], sum);
        q[h] = e[h] < E ? p[h] : -1.f;
    }
    int rank[2] = {kMaxE, kMaxE};
    for (int r = 0; r < k; ++r) {
        const float m = wave_max(fmaxf(q[0], q[1]));
        const uint64_t b0 = __ballot(q[0] == m), b1 = __ballot(q[1] == m);
        // the lowest expert index holding the maximum (experts 0..63 first);
        // none when the probabilities are not numbers
        const int win = b0 ? (int)__builtin_ctzll(b0) : (b1 ? 64 + (int)__builtin_ctzll(b1) : -1);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            if (win == e[h]) {
                rank[h] = r;
                q[h] = -INFINITY;
            }
    }
    bool sel[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) sel[h] = e[h] < E && rank[h] < k;
    const float den = fmaxf(wave_sum((sel[0] ? p[0] : 0.f) + (sel[1] ? p[1] : 0.f)), 1e-8f);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (e[h] >= E) continue;
        const int64_t pe = (int64_t)tok * E + e[h];
        if (sel[h]) {
            const int64_t at = (int64_t)tok * k + rank[h];
            o.topk_idx[at] = e[h];
            o.topk_w[at] = __fdiv_rn(p[h], den);
            if (sel_l) sel_l[at] = e[h];  // (LDS copy for a caller that goes on to the experts)
            atomicAdd(cnt_l + e[h], 1);
        }
        ps_w[e[h]] += p[h];
        if (o.probs) o.probs[pe] = p[h];
        if (o.mask) o.mask[pe] = sel[h] ? 1.f : 0.f;
        if (o.wdense) o.wdense[pe] = sel[h] ? __fdiv_rn(p[h], den) : 0.f;
    }
    if (o.y) {
        // the unselected experts' output blocks of the row, zeroed with the
        // lanes on consecutive 16-byte chunks (1 KB per store instruction,
        // whole cache lines; one lane per expert block wrote 16 bytes of 64
        // different lines per instruction, at a fraction of the HBM rate)
        const uint64_t s0 = __ballot(sel[0]), s1 = __ballot(sel[1]);
        const int cpb = o.y_bf16 ? 4 : 8;  // 16-byte chunks per 32-value block
        uint4 *row = (uint4 *)((char *)o.y + (int64_t)tok * o.ldy * (o.y_bf16 ? 2 : 4));
        for (int c = lane; c < E * cpb; c += 64) {
            const int ex = c / cpb;
            const bool chosen = ex < 64 ? (s0 >> ex) & 1u : (s1 >> (ex - 64)) & 1u;
            if (!chosen) row[c] = uint4{0, 0, 0, 0};
        }
    }
}

__global__ __launch_bounds__(kMoeThreads) void moe_topk_rank_kernel(const float *__restrict__ logits, RouteOut o) {
    __shared__ PartSums part;
    part_init(part);
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int tok = blockIdx.x * kMoeWaves + wave; tok < o.M; tok += gridDim.x * kMoeWaves) {
        float lg[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int e = lane + 64 * h;
            lg[h] = e < o.E ? logits[(int64_t)tok * o.E + e] : -INFINITY;
        }
        rank_token(tok, lg, o, part.cnt, part.ps[wave]);
    }
    part_store(part, o.count, o.probsum, o.E, o.n_part);
}

__global__ void moe_zero_kernel(int *count, float *probsum, int n) {
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        count[e] = 0;
        probsum[e] = 0.f;
    }
}

// ------------------------------------------------------------------ scatter
// moe_finalize_kernel (one workgroup of kFinSlices threads per expert):
// totals of the per-workgroup partial sums (each slice sums every
// kFinSlices-th row, 8 loads in flight, then the slices add in LDS),
// offset = exclusive scan of the counts, tile_off = exclusive scan of
// ceil(count / 16), cursor cleared.
constexpr int kFinSlices = 8;
// Totals, scans and cleared cursors (every thread of a kMaxE * kFinSlices
// workgroup); leaves the counts in c_s[0] and the offsets in off_s.
__device__ __forceinline__ void finalize_body(const int *__restrict__ count_part,
                                              const float *__restrict__ probsum_part, int n_part, int E,
                                              int *__restrict__ count, float *__restrict__ probsum,
                                              int *__restrict__ cursor, int *__restrict__ offset,
                                              int *__restrict__ tile_off, int (&c_s)[kFinSlices][kMaxE],
                                              float (&p_s)[kFinSlices][kMaxE], int *off_s) {
    const int e = threadIdx.x % kMaxE, sl = threadIdx.x / kMaxE;
    int c = 0;
    float ps = 0.f;
    if (e < E) {
        int r = sl;
        for (; r + 7 * kFinSlices < n_part; r += 8 * kFinSlices) {
            int cv[8];
            float pv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                cv[j] = count_part[(int64_t)(r + j * kFinSlices) * E + e];
                pv[j] = probsum_part[(int64_t)(r + j * kFinSlices) * E + e];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                c += cv[j];
                ps += pv[j];
            }
        }
        for (; r < n_part; r += kFinSlices) {
            c += count_part[(int64_t)r * E + e];
            ps += probsum_part[(int64_t)r * E + e];
        }
    }
    c_s[sl][e] = c;
    p_s[sl][e] = ps;
    __syncthreads();
    if (sl == 0) {
        for (int j = 1; j < kFinSlices; ++j) {
            c += c_s[j][e];
            ps += p_s[j][e];
        }
        if (e < E) {
            count[e] = c;
            probsum[e] = ps;
            cursor[e] = 0;
        }
        c_s[0][e] = e < E ? c : 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0, tacc = 0;
        for (int i = 0; i < E; ++i) {
            off_s[i] = acc;
            offset[i] = acc;
            tile_off[i] = tacc;
            acc += c_s[0][i];
            tacc += (c_s[0][i] + 15) / 16;
        }
        offset[E] = acc;
        tile_off[E] = tacc;
    }
}

__global__ __launch_bounds__(kMaxE * kFinSlices) void moe_finalize_kernel(const int *__restrict__ count_part,
                                                                          const float *__restrict__ probsum_part,
                                                                          int n_part, int E, int *__restrict__ count,
                                                                          float *__restrict__ probsum,
                                                                          int *__restrict__ cursor,
                                                                          int *__restrict__ offset,
                                                                          int *__restrict__ tile_off) {
    __shared__ int c_s[kFinSlices][kMaxE];
    __shared__ float p_s[kFinSlices][kMaxE];
    __shared__ int off_s[kMaxE];
    finalize_body(count_part, probsum_part, n_part, E, count, probsum, cursor, offset, tile_off, c_s, p_s, off_s);
}

// Few pairs (decode): the totals and the lists in one workgroup, the list
// ranks from LDS atomics; cursor ends at the counts, as after the
// two-launch form.
constexpr int kScatterSmallPairs = 4096;
__global__ __launch_bounds__(kMaxE * kFinSlices) void moe_scatter_small_kernel(
    const int *__restrict__ topk_idx, int n_pairs, const int *__restrict__ count_part,
    const float *__restrict__ probsum_part, int n_part, int E, int *__restrict__ count, float *__restrict__ probsum,
    int *__restrict__ cursor, int *__restrict__ offset, int *__restrict__ tile_off, int *__restrict__ list) {
    __shared__ int c_s[kFinSlices][kMaxE];
    __shared__ float p_s[kFinSlices][kMaxE];
    __shared__ int off_s[kMaxE];
    __shared__ int cur_s[kMaxE];
    if (threadIdx.x < kMaxE) cur_s[threadIdx.x] = 0;
    finalize_body(count_part, probsum_part, n_part, E, count, probsum, cursor, offset, tile_off, c_s, p_s, off_s);
    __syncthreads();  // offsets ready
    for (int p = threadIdx.x; p < n_pairs; p += blockDim.x) {
        const int e = topk_idx[p];
        if ((unsigned)e < (unsigned)E) list[off_s[e] + atomicAdd(&cur_s[e], 1)] = p;
    }
    __syncthreads();
    if (threadIdx.x < E) cursor[threadIdx.x] = cur_s[threadIdx.x];
}

// Each workgroup places a contiguous chunk of kScatterPerThread * 256 pairs:
// ranks inside the chunk come from LDS atomics, and one global atomic per
// (workgroup, expert) reserves the chunk's range of the expert's list.
constexpr int kScatterPerThread = 32;
__global__ __launch_bounds__(256) void moe_scatter_kernel(const int *__restrict__ topk_idx, int64_t n_pairs, int E,
                                                          const int *__restrict__ offset, int *__restrict__ cursor,
                                                          int *__restrict__ list) {
    __shared__ int hist[kMaxE], base[kMaxE];
    for (int e = threadIdx.x; e < kMaxE; e += 256) hist[e] = 0;
    __syncthreads();
    const int64_t p0 = (int64_t)blockIdx.x * 256 * kScatterPerThread;
    int ex[kScatterPerThread], rk[kScatterPerThread];
#pragma unroll
    for (int i = 0; i < kScatterPerThread; ++i) {
        const int64_t p = p0 + (int64_t)i * 256 + threadIdx.x;
        const int e = p < n_pairs ? topk_idx[p] : -1;
        ex[i] = (unsigned)e < (unsigned)E ? e : -1;
    }
#pragma unroll
    for (int i = 0; i < kScatterPerThread; ++i) rk[i] = ex[i] >= 0 ? atomicAdd(&hist[ex[i]], 1) : 0;
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 256) base[e] = hist[e] ? offset[e] + atomicAdd(cursor + e, hist[e]) : 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kScatterPerThread; ++i)
        if (ex[i] >= 0) list[base[ex[i]] + rk[i]] = (int)(p0 + (int64_t)i * 256 + threadIdx.x);
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

// Code byte -> its 4 ternary values as floats (the MFMA A-operand table).
__device__ __forceinline__ void expert_lut_init(f32x4 *lut) {
    for (uint32_t byte = threadIdx.x; byte < 256; byte += blockDim.x) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (float)((int)((byte >> (6 - 2 * j)) & 3u) - 1);
        lut[byte] = v;
    }
}

// One wavefront's item: expert e for up to 16 routed pairs, lane column t
// holding pair `pair` (ok: the column is in use).  gate/up as D[hidden][pair],
// silu(g) * u, then down; y[tok, 32e:32e+32] = expert output * routing
// weight.  Every column is computed on its own, so a pair's result does not
// depend on which item or column it lands in.
// PRELOAD: every code byte of the item is requested before the first
// product (one memory round trip; for a launch whose item is its critical
// path), instead of as the products go.
template <typename T, typename TY, bool BF16MMA, int NHT, bool PRELOAD = false>
__device__ __forceinline__ void expert_item(const ExpArgs &a, const f32x4 *lut, __amdgpu_buffer_rsrc_t xr,
                                            __amdgpu_buffer_rsrc_t yr, int e, int pair, bool ok) {
    constexpr uint32_t esz = sizeof(T);
    constexpr int nht = NHT;  // hidden tiles of 16 (H = 16 * NHT)
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const float gg = a.gammas[0], gu = a.gammas[1], gd = a.gammas[2];
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
    const uint8_t *df = a.down_f + (int64_t)e * nht * 128;
    uint32_t gb[PRELOAD ? 2 * NHT : 1], ub[PRELOAD ? 2 * NHT : 1], db[PRELOAD ? 2 * NHT : 1];
    if constexpr (PRELOAD) {
#pragma unroll
        for (int i = 0; i < 2 * nht; ++i) {
            gb[i] = gf[i * 64 + lane];
            ub[i] = uf[i * 64 + lane];
        }
#pragma unroll
        for (int i = 0; i < 2 * nht; ++i) db[i] = df[i * 64 + lane];
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int nt = 0; nt < nht; ++nt) {
        f32x4 g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            g = mma16<BF16MMA>(lut[PRELOAD ? gb[nt * 2 + c] : gf[(nt * 2 + c) * 64 + lane]], xb[c], g);
            u = mma16<BF16MMA>(lut[PRELOAD ? ub[nt * 2 + c] : uf[(nt * 2 + c) * 64 + lane]], xb[c], u);
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
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < nht; ++ks)
            d = mma16<BF16MMA>(lut[PRELOAD ? db[mt * nht + ks] : df[(mt * nht + ks) * 64 + lane]], hb[ks], d);
        f32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = (BF16MMA ? bf16r(gd * d[j]) : gd * d[j]) * wr;
        Buf4<TY>::store(o, yr,
                        xo == kOOB ? kOOB : (uint32_t)(((int64_t)tok * a.ldy + 32 * e + 16 * mt + 4 * q) * sizeof(TY)),
                        0);
    }
}

template <typename T, typename TY, bool BF16MMA, int NHT>
__global__ __launch_bounds__(kMoeThreads, 2) void moe_experts_kernel(ExpArgs a) {
    __shared__ __align__(16) f32x4 lut[256];
    __shared__ int toff[129];
    expert_lut_init(lut);
    for (int e = threadIdx.x; e <= a.E; e += kMoeThreads) toff[e] = a.tile_off[e];
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = lane & 15;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * sizeof(T)));
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
        expert_item<T, TY, BF16MMA, NHT>(a, lut, xr, yr, e, pair, ok);
    }
}

// ------------------------------------------------------------------ fused FFN
// The whole HadamardMoE.forward (moe.py:512-542) for n_embd 512 (16 experts,
// router 512 -> 128 -> 16) in one persistent kernel, bf16 operands on the
// matrix cores.  A workgroup (8 waves, two per SIMD so that one wave's
// matrix-core and memory waits overlap the other's VALU work) takes 64
// tokens at a time:
//   0. the 64 x 512 input tile is copied to LDS (the only HBM read of x),
//      its rows requested in 16-token sub-tiles behind the wave's W1 rows;
//   1. as each sub-tile lands (the later ones still in flight), wave w
//      computes router hidden units 16w..16w+15 for its 16 tokens, applies
//      silu and forms its partial logits over those 16 units;
//   2. waves 0-3 each sum the 8 partial logits of 16 tokens (fixed order)
//      and route them (softmax, top-k, weights): routing outputs, and a
//      per-token selection mask and weights in LDS;
//   3. wave w runs experts w and w+8: it zeroes the expert's output blocks
//      of the tokens that did not choose it, then a ballot over the 64
//      tokens' masks and a prefix count compact the tokens that did, which
//      are processed 16 at a time (gate/up, silu, down) with x read back
//      from LDS; outputs go straight to y (blocks are disjoint).
// Per-expert counts accumulate in LDS (integer atomics), probability sums
// in a fixed order (DPP row shifts and row swaps within a routing wave, the
// four waves' rows in order), so they are the same on every run; each
// workgroup stores its partial sums in its own row (same-address global
// atomics from every workgroup would serialise across the chip).
constexpr int kFfnC = 512, kFfnE = 16, kFfnTok = 64, kFfnWaves = 8, kFfnThreads = 64 * kFfnWaves;
constexpr int kXsStride = kFfnC * 2 + 16;  // bytes per token row of the LDS tile (padded)

__device__ __forceinline__ f32x4 mma32(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ f32x4 mma16bf(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c,
                                                     0, 0, 0);
}

// 8 ternary codes (two packed bytes, low byte first) -> 8 bf16.
__device__ __forceinline__ uint4 decode8(const uint2 *lut, uint32_t u16) {
    const uint2 lo = lut[u16 & 0xffu], hi = lut[(u16 >> 8) & 0xffu];
    return uint4{lo.x, lo.y, hi.x, hi.y};
}

// NH (multiple of 4) consecutive 16-bit code pairs as NH/2 words, 8 bytes
// per load; code pair i is (w[i / 2] >> (16 * (i % 2))) (decode8 masks).
template <int NH>
__device__ __forceinline__ void load_codes(const uint16_t *p, uint32_t (&w)[NH / 2]) {
#pragma unroll
    for (int i = 0; i < NH / 4; ++i) {
        const uint2 v = *(const uint2 *)(p + 4 * i);
        w[2 * i] = v.x;
        w[2 * i + 1] = v.y;
    }
}

template <int NH>
__device__ __forceinline__ uint32_t code_pair(const uint32_t (&w)[NH / 2], int i) {
    return w[i >> 1] >> (16 * (i & 1));
}

struct FfnArgs {
    const uint16_t *x;
    int64_t ldx;
    int M, k;
    const uint4 *w1f;         // [8 nt][16 ks][64]: W1[16nt + l%16][32ks + 8(l/16) + s], s < 8
    const uint2 *w2f;         // [8 c][64]: W2[l%16][16c + 4(l/16) + s], s < 4 (rows >= E zero)
    const uint16_t *gate_f;   // [16][64][NH]: packed bytes 2(l/16), 2(l/16)+1 of row 16nt + l%16
    const uint16_t *up_f;     // [16][64][NH]
    const uint16_t *down_f;   // [16][64][2][NH/2]: bytes 8c + l/16, 8c + 4 + l/16 of row 16mt + l%16
    const float *gammas;
    int *topk_idx;
    float *topk_w;
    int *count;       // [n_part][16] per-workgroup partial counts
    float *probsum;   // [n_part][16]
    int n_part;
    void *y;
    int64_t ldy;
};

template <typename TY, int NH>
__global__ __launch_bounds__(kFfnThreads, 1) void moe_ffn_kernel(FfnArgs a) {
    __shared__ __align__(16) uint8_t xs[kFfnTok * kXsStride];
    __shared__ __align__(16) f32x4 lp[kFfnWaves][kFfnTok][4];  // partial logits [wave][token][q]
    __shared__ __align__(16) float ws[kFfnTok][kFfnE];         // routing weights (0 = unselected)
    __shared__ uint32_t sel_s[kFfnTok];                        // bit e: token chose expert e
    __shared__ int list_s[kFfnWaves][kFfnTok];
    __shared__ uint2 lut[256];
    __shared__ int cnt_s[kFfnE];
    __shared__ float ps_s[kFfnE];                              // written by thread e only
    __shared__ __align__(16) float ps_w[4][kFfnE];             // per routing wave, per tile
    static_assert(NH <= 8, "hidden <= 128");
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int t = lane & 15, q = lane >> 4;
    if (tid < 256) {
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int v0 = (int)((tid >> (6 - 4 * h)) & 3u) - 1, v1 = (int)((tid >> (4 - 4 * h)) & 3u) - 1;
            const uint32_t b0 = v0 == 0 ? 0u : (v0 > 0 ? 0x3f80u : 0xbf80u);
            const uint32_t b1 = v1 == 0 ? 0u : (v1 > 0 ? 0x3f80u : 0xbf80u);
            w[h] = b0 | (b1 << 16);
        }
        lut[tid] = uint2{w[0], w[1]};
    }
    if (tid < kFfnE) {
        cnt_s[tid] = 0;
        ps_s[tid] = 0.f;
    }
    const int M = a.M;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)M * a.ldx * 2));
    // silu(gg g) * (gu u) = gg gu * [g / (1 + exp(-gg g))] * u: the exp
    // argument carries gg (with log2 e), the down scale carries gg gu gd
    const float gg = a.gammas[0], gu = a.gammas[1], gd = a.gammas[2];
    const float kexp = -gg * 1.4426950408889634f, gdown = gd * gg * gu;
    const int ybf = sizeof(TY) == 2;

    for (int base = blockIdx.x * kFfnTok; base < M; base += gridDim.x * kFfnTok) {
        lds_barrier();  // the previous tile is no longer read
        // 0. this wave's router rows first (L2-resident: the x rows queue
        //    behind them), then the input tile's rows (past M: zeros), wave
        //    w taking rows 8i + w, so the rows of 16-token sub-tile s (i = 2s,
        //    2s + 1) land in sub-tile order; then this wave's expert codes
        //    (w, w + 8), decoded in phase 3.  (All reloaded per tile: kept
        //    across the expert phase they would take its registers.)
        uint4 w1r[kFfnC / 32];
#pragma unroll
        for (int ks = 0; ks < kFfnC / 32; ++ks) w1r[ks] = a.w1f[(wave * 16 + ks) * 64 + lane];
        const uint2 w2 = a.w2f[wave * 64 + lane];
        uint4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 8 * i + wave, c = lane;
            const uint32_t off = base + r < M ? (uint32_t)(((int64_t)(base + r) * a.ldx + 8 * c) * 2) : kOOB;
            v[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        }
        uint32_t cg[2][NH / 2], cu[2][NH / 2], cd[2][NH / 2];
#pragma unroll
        for (int x2 = 0; x2 < 2; ++x2) {
            const int64_t off = ((int64_t)(wave + kFfnWaves * x2) * 64 + lane) * NH;
            load_codes<NH>(a.gate_f + off, cg[x2]);
            load_codes<NH>(a.up_f + off, cu[x2]);
            load_codes<NH>(a.down_f + off, cd[x2]);
        }
        // 1. per sub-tile, as its rows land (the later sub-tiles still in
        //    flight): router hidden units 16w..16w+15 of its 16 tokens, then
        //    this wave's partial logits
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
#pragma unroll
            for (int i = 2 * sub; i < 2 * sub + 2; ++i)
                *(uint4 *)(xs + (8 * i + wave) * kXsStride + 16 * lane) = v[i];
            lds_barrier();
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < kFfnC / 32; ++ks) {
                const uint4 b = *(const uint4 *)(xs + (16 * sub + t) * kXsStride + (32 * ks + 8 * q) * 2);
                acc = mma32(w1r[ks], b, acc);
            }
            float h[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) h[j] = silu_f(bf16r(acc[j]));
            const uint2 hb{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
            lp[wave][16 * sub + t][q] = mma16bf(w2, hb, f32x4{0.f, 0.f, 0.f, 0.f});
        }
        lds_barrier();
        // 2. routing of tokens 16w..16w+15 (waves 0-3).  Lane l takes token
        //    16w + l / 4 and experts 4 (l % 4) .. +3: a token's four lanes
        //    form a DPP quad, so the top-k exchanges stay in the VALU
        if (wave < 4) {
            const int rq = lane & 3, tl = 16 * wave + (lane >> 2), tok = base + tl;
            const bool tok_ok = tok < M;
            f32x4 sl = lp[0][tl][rq];
#pragma unroll
            for (int w = 1; w < kFfnWaves; ++w) sl += lp[w][tl][rq];
            float lg[1][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) lg[0][j] = bf16r(sl[j]);
            TopK<1> r;
            topk_core<1, 1, 2>(lg, 1, kFfnE, a.k, rq, r);
            f32x4 wv, pv;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool sj = tok_ok && ((r.sel[0] >> j) & 1u);
                wv[j] = sj ? __fdiv_rn(r.p[0][j], r.den) : 0.f;
                if (sj) {
                    const int64_t at = (int64_t)tok * a.k + r.rank[0][j];
                    a.topk_idx[at] = 4 * rq + j;
                    a.topk_w[at] = wv[j];
                }
                if (sj) atomicAdd(&cnt_s[4 * rq + j], 1);
                pv[j] = tok_ok ? r.p[0][j] : 0.f;
            }
            *(f32x4 *)&ws[tl][4 * rq] = wv;
            // the wave's probability sums per expert in a fixed order: the 4
            // tokens of each 16-lane row (DPP row shifts by 4 and 8, ending
            // in lanes 12..15), then the 4 rows (row and half swaps)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v = pv[j];
                v += row_shr<4>(v);
                v += row_shr<8>(v);
                const u32x2 h1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
                v = __uint_as_float(h1.x) + __uint_as_float(h1.y);
                const u32x2 h2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
                pv[j] = __uint_as_float(h2.x) + __uint_as_float(h2.y);
            }
            if (lane >= 12 && lane < 16) *(f32x4 *)&ps_w[wave][4 * rq] = pv;
            uint32_t m = tok_ok ? (r.sel[0] & 15u) << (4 * rq) : 0u;
            m |= (uint32_t)xchg_i<1>((int)m);
            m |= (uint32_t)xchg_i<2>((int)m);
            if (rq == 0) sel_s[tl] = m;
        }
        lds_barrier();
        // this tile's probability sums: the four routing waves' rows in order
        if (tid < kFfnE) ps_s[tid] += ((ps_w[0][tid] + ps_w[1][tid]) + ps_w[2][tid]) + ps_w[3][tid];
        // 3. experts w and w + 8 on the tokens that chose them.  (Taking
        //    (expert, group) items from a counter, with every expert's codes
        //    in LDS, balanced the waves but ran slower: the expert phase is
        //    bound by the SIMDs' VALU work, which that does not reduce.)
#pragma unroll
        for (int x2 = 0; x2 < 2; ++x2) {
            const int e = wave + kFfnWaves * x2;
            const uint32_t tsel = sel_s[lane];
            const bool mine = (tsel >> e) & 1u;
            const uint64_t bal = __ballot(mine);
            // zero the blocks of the tile's tokens that did not choose e (their
            // stores overlap this wave's expert arithmetic): 8 (fp32) or 4
            // (bf16) lanes per token block, so each store instruction writes
            // whole blocks (128 / 64 contiguous bytes) of 8 or 16 tokens
            {
                const int per = ybf ? 4 : 8, rows = 64 / per;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (ybf && i >= 4) break;
                    const int tl = rows * i + lane / per, tok = base + tl;
                    if (tok < M && !((bal >> tl) & 1ull)) {
                        const int64_t at = (int64_t)tok * a.ldy + 32 * e;
                        uint4 *d = ybf ? (uint4 *)((uint16_t *)a.y + at) : (uint4 *)((float *)a.y + at);
                        d[lane % per] = uint4{0, 0, 0, 0};
                    }
                }
            }
            const int n = __popcll(bal);
            if (mine) {
                const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                list_s[wave][rank] = lane;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (n == 0) continue;
            // the expert's weights as bf16 operands, decoded once for all its groups
            uint4 ag[NH], au[NH], ad[NH];
#pragma unroll
            for (int i = 0; i < NH; ++i) {
                ag[i] = decode8(lut, code_pair<NH>(cg[x2], i));
                au[i] = decode8(lut, code_pair<NH>(cu[x2], i));
                ad[i] = decode8(lut, code_pair<NH>(cd[x2], i));
            }
            for (int g = 0; g < n; g += 16) {
                const bool ok = g + t < n;
                const int tl = ok ? list_s[wave][g + t] : 0;
                const uint4 xb = ok ? *(const uint4 *)(xs + tl * kXsStride + (32 * e + 8 * q) * 2) : uint4{0, 0, 0, 0};
                const float wr = ok ? ws[tl][e] : 0.f;
                uint4 hb[NH / 2];
#pragma unroll
                for (int c = 0; c < NH / 2; ++c) {
                    float hv[2][4];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const f32x4 z{0.f, 0.f, 0.f, 0.f};
                        const f32x4 gv = mma32(ag[2 * c + h], xb, z);
                        const f32x4 uv = mma32(au[2 * c + h], xb, z);
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            hv[h][j] = gv[j] * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(kexp * gv[j])) * uv[j];
                    }
                    hb[c] = uint4{pack_bf16x2(hv[0][0], hv[0][1]), pack_bf16x2(hv[0][2], hv[0][3]),
                                  pack_bf16x2(hv[1][0], hv[1][1]), pack_bf16x2(hv[1][2], hv[1][3])};
                }
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    f32x4 d{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < NH / 2; ++c) d = mma32(ad[mt * (NH / 2) + c], hb[c], d);
                    if (ok) {
                        f32x4 o;
#pragma unroll
                        for (int j = 0; j < 4; ++j) o[j] = bf16r(gdown * d[j]) * wr;
                        const int64_t at = (int64_t)(base + tl) * a.ldy + 32 * e + 16 * mt + 4 * q;
                        store4((TY *)a.y + at, o);
                    }
                }
            }
        }
    }
    lds_barrier();
    if (tid < kFfnE) {
        a.count[blockIdx.x * kFfnE + tid] = cnt_s[tid];
        a.probsum[blockIdx.x * kFfnE + tid] = ps_s[tid];
        for (int r = blockIdx.x + gridDim.x; r < a.n_part; r += gridDim.x) {
            a.count[r * kFfnE + tid] = 0;
            a.probsum[r * kFfnE + tid] = 0.f;
        }
    }
}

}  // namespace walsh

using namespace walsh;

static int grid_cap(int64_t waves_needed, int64_t limit = 0) {
    int64_t g = ceil_div(waves_needed, kMoeWaves);
    const int64_t cap = (int64_t)device_info().cu_count * 4;
    if (g > cap) g = cap;
    if (limit > 0 && g > limit) g = limit;
    return (int)(g < 1 ? 1 : g);
}

// ------------------------------------------------------------------ wide router
// The router of wide models (n_embd above the fused router's limit, e.g.
// 4096 -> 1024 -> 128 experts; moe.py:407-447) as two launches on bf16
// matrix cores:
//   1. h = silu(x W1^T) [M, H] into a caller workspace: the 256 x 256-tile
//      GEMM at many rows; at few rows (decode) router_w1_small_kernel, one
//      workgroup per 16 hidden units x 16 tokens whose 8 waves split K, and
//      which also forms its 16 hidden units' share of every logit (a
//      16x16x16 product per 16 experts) into partial sums [H/16][M][E];
//   2. many rows: router_w2_topk_kernel, logits = h W2^T for 64 tokens per
//      workgroup (the tile of h staged in LDS, wave w taking experts
//      16w..16w+15); few rows: router_topk_part_kernel adds the H/16
//      partial sums in order; then softmax / rank top-k / routing outputs
//      per token as in walsh_moe_topk_fwd.
// Products are rounded to bf16 where the reference's autocast Linears round
// their outputs, with SiLU on the rounded first product.
constexpr int kR1Waves = 8;
constexpr int kR1SmallRows = 256;  // row counts up to this take the split-K kernel
// CPOL: cache policy of the partial-logit stores (16: device scope, sc1, for
// a reader in another workgroup of the same launch).
template <int CPOL = 0>
__device__ __forceinline__ void router_w1_small_body(const uint16_t *__restrict__ x, int64_t ldx, int M, int C,
                                                     const uint16_t *__restrict__ w1, uint16_t *__restrict__ h,
                                                     int64_t ldh, const uint16_t *__restrict__ w2, int E,
                                                     float *__restrict__ lpart, f32x4 (*part)[64]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, fr = lane & 15, fq = lane >> 4;
    const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16, H = gridDim.x * 16;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)((int64_t)M * ldx * 2));
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w1, (uint32_t)((int64_t)H * C * 2));
    // wave w: columns [w C/8, (w+1) C/8) in 32-column steps, 8 steps of
    // operands in flight
    const int kw = C / kR1Waves, k0 = wave * kw;
    const uint32_t wo = (uint32_t)(((int64_t)(n0 + fr) * C + k0 + 8 * fq) * 2);
    // wave 0's W2 fragments for the partial logits, in flight from the start
    const __amdgpu_buffer_rsrc_t w2r = make_rsrc(w2, (uint32_t)((int64_t)E * H * 2));
    u32x2 a2[kMaxE / 16];
#pragma unroll
    for (int et = 0; et < kMaxE / 16; ++et) {
        const int e = 16 * et + fr;
        a2[et] = __builtin_amdgcn_raw_buffer_load_b64(
            w2r, (wave == 0 && e < E) ? (uint32_t)(((int64_t)e * H + n0 + 4 * fq) * 2) : kOOB, 0, 0);
    }
    const bool row_ok = m0 + fr < M;
    const uint32_t xo = row_ok ? (uint32_t)(((int64_t)(m0 + fr) * ldx + k0 + 8 * fq) * 2) : 0;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kk = 0; kk < kw; kk += 8 * 32) {
        u32x4 a[8], b[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = kk + 32 * j;
            a[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, k < kw ? wo + (uint32_t)k * 2 : kOOB, 0, 0);
            b[j] = __builtin_amdgcn_raw_buffer_load_b128(xr, (k < kw && row_ok) ? xo + (uint32_t)k * 2 : kOOB, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[j]),
                                                          __builtin_bit_cast(bf16x8, b[j]), acc, 0, 0, 0);
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave) return;  // waves 1.. leave the body here; wave 0 finishes it
    f32x4 v = part[0][lane];
#pragma unroll
    for (int w = 1; w < kR1Waves; ++w) v = v + part[w][lane];
    // lane holds D[n = n0 + 4 fq + r][m = m0 + fr]
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = silu_f(bf16r(v[r]));
    const __amdgpu_buffer_rsrc_t hr = make_rsrc(h, (uint32_t)((int64_t)M * ldh * 2));
    Buf4<uint16_t>::store(v, hr, row_ok ? (uint32_t)(((int64_t)(m0 + fr) * ldh + n0 + 4 * fq) * 2) : kOOB, 0);
    // these 16 hidden units' share of the logits: lane (fr, fq) holds the
    // B operand of a 16x16x16 product (hidden n0 + 4 fq .. +3 of token
    // m0 + fr); A = W2[16 et + fr][n0 + 4 fq .. +3]
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(lpart + (int64_t)blockIdx.x * M * E, (uint32_t)((int64_t)M * E * 4));
    const u32x2 b = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
#pragma unroll
    for (int et = 0; et < kMaxE / 16; ++et) {
        const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a2[et]),
                                                                 __builtin_bit_cast(i16x4, b),
                                                                 f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        // d[r] = partial logit of expert 16 et + 4 fq + r for token m0 + fr
        // (E % 4 == 0: the 4 experts are valid together)
        const int e0 = 16 * et + 4 * fq;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, d), pr,
                                               (row_ok && e0 < E) ? (uint32_t)(((int64_t)(m0 + fr) * E + e0) * 4) : kOOB,
                                               0, CPOL);
    }
}

__global__ __launch_bounds__(64 * kR1Waves) void router_w1_small_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                                        int M, int C, const uint16_t *__restrict__ w1,
                                                                        uint16_t *__restrict__ h, int64_t ldh,
                                                                        const uint16_t *__restrict__ w2, int E,
                                                                        float *__restrict__ lpart) {
    __shared__ f32x4 part[kR1Waves][64];
    router_w1_small_body(x, ldx, M, C, w1, h, ldh, w2, E, lpart, part);
}

// Few rows: logits = the H/16 partial sums of router_w1_small_kernel added
// in a fixed order (wave w sums partials 16w..16w+15, then the 4 wave sums
// in wave order), rounded to bf16; then wave 0 routes the token.
constexpr int kTopkPartMax = 64;  // H / 16 <= 64
__global__ __launch_bounds__(kMoeThreads) void router_topk_part_kernel(const float *__restrict__ lpart, int nparts,
                                                                       RouteOut o) {
    __shared__ PartSums part;
    __shared__ __align__(16) float ws[kMoeWaves][kMaxE];
    part_init(part);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int E = o.E, M = o.M;
    constexpr int kPer = kTopkPartMax / kMoeWaves;
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(lpart, (uint32_t)((int64_t)nparts * M * E * 4));
    const int e = 2 * lane;  // lane: experts 2 lane, 2 lane + 1 (one 8-byte load per partial)
    for (int tok = blockIdx.x; tok < M; tok += gridDim.x) {
        u32x2 pv[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int jj = wave * kPer + j;
            pv[j] = __builtin_amdgcn_raw_buffer_load_b64(
                pr, (e < E && jj < nparts) ? (uint32_t)((((int64_t)jj * M + tok) * E + e) * 4) : kOOB, 0, 0);
        }
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            acc0 += __uint_as_float(pv[j].x);
            acc1 += __uint_as_float(pv[j].y);
        }
        __syncthreads();  // the previous token's ws is read
        *(f32x2 *)&ws[wave][e] = f32x2{acc0, acc1};
        __syncthreads();
        if (wave == 0) {
            float lg[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int ee = lane + 64 * hh;
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < kMoeWaves; ++w) v += ws[w][ee];
                lg[hh] = ee < E ? bf16r(v) : -INFINITY;
            }
            rank_token(tok, lg, o, part.cnt, part.ps[wave]);
        }
    }
    part_store(part, o.count, o.probsum, o.E, o.n_part);
}

constexpr int kR2Waves = 8;    // wave w: experts 16w..16w+15
constexpr int kR2MaxH = 1024;  // staged tile of h: up to 64 x 1024 bf16 = 128 KB of LDS
constexpr int kR2LgStride = kMaxE + 4;

// TT 16-token tiles per workgroup: 4 (64 tokens) for many rows, 1 for a
// decode-sized batch (a quarter of the staging and the products)
static size_t router_w2_lds_bytes(int H, int TT) {
    const size_t stage = (size_t)16 * TT * H * 2, lg = (size_t)16 * TT * kR2LgStride * 4;
    return stage > lg ? stage : lg;
}

// smem: the h tile, 16-byte chunk c of row r at r * 2H + ((c ^ (r & 15)) << 4)
// (the 16 rows of a fragment read fall on 16 different chunk columns); after
// the products the rounded logits [64][kR2LgStride] float.
template <int TT>
__global__ __launch_bounds__(64 * kR2Waves) void router_w2_topk_kernel(const uint16_t *__restrict__ h, int64_t ldh,
                                                                       int H, const uint16_t *__restrict__ w2,
                                                                       RouteOut o) {
    constexpr int kR2Tok = 16 * TT;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ PartSums part;
    part_init(part);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, fr = lane & 15, fq = lane >> 4;
    const int M = o.M, E = o.E, nch = H / 8, nks = H / 32;
    const __amdgpu_buffer_rsrc_t hr = make_rsrc(h, (uint32_t)((int64_t)M * ldh * 2));
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w2, (uint32_t)((int64_t)E * H * 2));
    const int e_row = 16 * wave + fr;
    const uint32_t wo = e_row < E ? (uint32_t)(((int64_t)e_row * H + 8 * fq) * 2) : kOOB;
    float *lg_l = (float *)smem;
    const int n_tiles = (int)ceil_div(M, kR2Tok);
    for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const int m0 = tile * kR2Tok;
        // the first half of this wave's W2 fragments and the whole h tile in
        // flight together
        u32x4 wa[16];
#pragma unroll
        for (int s = 0; s < 16; ++s)
            wa[s] = __builtin_amdgcn_raw_buffer_load_b128(wr, (s < nks && wo != kOOB) ? wo + (uint32_t)s * 64 : kOOB,
                                                          0, 0);
        u32x4 st[kR2Tok * kR2MaxH / 8 / (64 * kR2Waves)];  // TT * 4 chunks per thread
#pragma unroll
        for (int j = 0; j < kR2Tok * kR2MaxH / 8 / (64 * kR2Waves); ++j) {
            const int i = tid + j * 64 * kR2Waves, r = i / nch, c = i - r * nch;
            const bool ok = i < kR2Tok * nch && m0 + r < M;
            st[j] = __builtin_amdgcn_raw_buffer_load_b128(
                hr, ok ? (uint32_t)(((int64_t)(m0 + r) * ldh + 8 * c) * 2) : kOOB, 0, 0);
        }
        __syncthreads();  // the previous tile's logits are read
#pragma unroll
        for (int j = 0; j < kR2Tok * kR2MaxH / 8 / (64 * kR2Waves); ++j) {
            const int i = tid + j * 64 * kR2Waves, r = i / nch, c = i - r * nch;
            if (i < kR2Tok * nch) *(u32x4 *)(smem + r * 2 * H + ((c ^ (r & 15)) << 4)) = st[j];
        }
        __syncthreads();
        f32x4 acc[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < nks; s0 += 16) {
            u32x4 wn[16];
            const bool more = s0 + 16 < nks;
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int sn = s0 + 16 + s;
                wn[s] = __builtin_amdgcn_raw_buffer_load_b128(
                    wr, (more && sn < nks && wo != kOOB) ? wo + (uint32_t)sn * 64 : kOOB, 0, 0);
            }
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                if (s0 + s < nks) {
                    const int c = 4 * (s0 + s) + fq;
#pragma unroll
                    for (int t = 0; t < TT; ++t) {
                        const int r = 16 * t + fr;
                        const u32x4 b = *(const u32x4 *)(smem + r * 2 * H + ((c ^ (r & 15)) << 4));
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wa[s]),
                                                                         __builtin_bit_cast(bf16x8, b), acc[t], 0, 0,
                                                                         0);
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < 16; ++s) wa[s] = wn[s];
        }
        __syncthreads();  // every wave is done with the h tile
        // acc[t][r] = logit of expert 16 w + 4 fq + r for token m0 + 16 t + fr
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            f32x4 v;
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = bf16r(acc[t][r]);
            *(f32x4 *)(lg_l + (16 * t + fr) * kR2LgStride + 16 * wave + 4 * fq) = v;
        }
        __syncthreads();
        for (int tl = wave; tl < kR2Tok && m0 + tl < M; tl += kR2Waves) {
            float lg[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int e = lane + 64 * hh;
                lg[hh] = e < E ? lg_l[tl * kR2LgStride + e] : -INFINITY;
            }
            rank_token(m0 + tl, lg, o, part.cnt, part.ps[wave]);
        }
    }
    part_store(part, o.count, o.probsum, o.E, o.n_part);
}

// ------------------------------------------------------------------ decode-sized MoE
// The whole HadamardMoE.forward (moe.py:512-542) of a wide model for a few
// tokens (decode) in one launch.  The H/16 workgroups of
// router_w1_small_kernel compute the router's hidden units and their shares
// of the logits; each then counts itself done on a counter, and the last one
// (release / acquire fences at device scope around the count) adds the
// partial logits in router_topk_part_kernel's order, routes every token
// (rank_token), lists the routed pairs by expert and runs the experts
// (expert_item, one wavefront per expert), so every output is bitwise the
// four-launch path's.  The counter is the caller's and starts at zero; the
// last workgroup sets it back to zero.
constexpr int kDecTok = 4;                       // tokens a launch takes
constexpr int kDecPairs = kDecTok * kMaxK;       // routed pairs at most

template <typename TY, int NHT>
__global__ __launch_bounds__(64 * kR1Waves) void moe_decode_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                                   int C, const uint16_t *__restrict__ w1,
                                                                   uint16_t *__restrict__ h,
                                                                   const uint16_t *__restrict__ w2,
                                                                   float *__restrict__ lpart, RouteOut o, ExpArgs ex,
                                                                   unsigned *__restrict__ sync) {
    __shared__ f32x4 part[kR1Waves][64];
    __shared__ int cnt_l[kDecTok][kMaxE];
    __shared__ float ps_l[kDecTok][kMaxE];
    __shared__ __align__(16) f32x4 lut[256];
    __shared__ int item_e[kDecPairs], item_n[kDecPairs], item_p[kDecPairs][kDecTok];
    __shared__ int sel_l[kDecPairs];
    __shared__ int n_items;
    __shared__ int last;
    __shared__ float gsum_l[kDecTok][4][kMaxE];  // group sums of the partial logits
    const int M = o.M, E = o.E, H = (int)gridDim.x * 16;
    // The hand-off without device-scope fences (whose L2 write-back and
    // invalidation cost microseconds here): wave 0 stores the partial logits
    // at device scope (sc1: performed at the point every XCD's accesses meet),
    // waits until they are acknowledged, then counts; the last workgroup
    // reads them with device-scope loads issued after its count returned.
    router_w1_small_body<16>(x, ldx, M, C, w1, h, H, w2, E, lpart, part);
    if (threadIdx.x == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial-logit stores are performed
        last = __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nparts = (int)gridDim.x;  // H / 16 <= kTopkPartMax
    // the partial logits added as router_topk_part_kernel adds them: groups
    // of 16 partials (zeros past nparts) in order, then the 4 group sums in
    // order.  Wave w forms group w % 4 of the experts lane + 64 (w / 4) for
    // every token, its loads requested before the LDS set-up below; wave
    // t < M then adds token t's group sums.
    const int grp = wave & 3, ge = lane + 64 * (wave >> 2);
    float pv[kDecTok][16];
    {
        const __amdgpu_buffer_rsrc_t pr = make_rsrc(lpart, (uint32_t)((int64_t)nparts * M * E * 4));
#pragma unroll
        for (int t = 0; t < kDecTok; ++t) {
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int j = 16 * grp + u;
                pv[t][u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    pr, (t < M && ge < E && j < nparts) ? (uint32_t)((((int64_t)j * M + t) * E + ge) * 4) : kOOB, 0,
                    16));  // device scope (sc1)
            }
        }
    }
    for (int i = threadIdx.x; i < kDecTok * kMaxE; i += blockDim.x) {
        cnt_l[i / kMaxE][i % kMaxE] = 0;
        ps_l[i / kMaxE][i % kMaxE] = 0.f;
    }
    for (int i = threadIdx.x; i < kDecPairs; i += blockDim.x) sel_l[i] = -1;  // slots no token fills stay -1
    expert_lut_init(lut);
#pragma unroll
    for (int t = 0; t < kDecTok; ++t) {
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < 16; ++u) acc += pv[t][u];
        gsum_l[t][grp][ge] = acc;
    }
    __syncthreads();
    if (wave < M) {
        const int tok = wave;
        float lg[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int e = lane + 64 * hh;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < kTopkPartMax / 16; ++w) v += gsum_l[tok][w][e];
            lg[hh] = e < E ? bf16r(v) : -INFINITY;
        }
        rank_token(tok, lg, o, cnt_l[tok], ps_l[tok], sel_l);
    }
    __syncthreads();  // routing outputs and the LDS rows are complete
    // partial-count rows: row t holds token t's counts and probabilities (as
    // router_topk_part_kernel's workgroup per token writes them), rows past
    // M zero
    for (int i = threadIdx.x; i < o.n_part * E; i += blockDim.x) {
        const int r = i / E, e = i % E;
        o.count[i] = r < M ? cnt_l[r][e] : 0;
        o.probsum[i] = r < M ? ps_l[r][e] : 0.f;
    }
    if (wave == 0) {
        // the routed pairs grouped by expert, in pair order (at most
        // kDecPairs <= 64, lane p holding pair p): each round takes the
        // expert of the lowest pair not yet listed (experts in order of first
        // appearance) and lists every pair of that expert
        const int ep = lane < M * o.k ? sel_l[lane] : -1;
        // (probabilities that are not numbers select fewer than k)
        const bool valid = ep >= 0 && ep < E;
        uint64_t pending = __ballot(valid);
        int n = 0;
        while (pending) {
            const int lead = (int)__builtin_ctzll(pending);
            const int el = __builtin_amdgcn_readlane(ep, lead);
            const uint64_t same = __ballot(valid && ep == el);
            if ((same >> lane) & 1u) item_p[n][__builtin_popcountll(same & ((1ull << lane) - 1))] = lane;
            if (lane == 0) {
                item_e[n] = el;
                item_n[n] = __builtin_popcountll(same);
            }
            pending &= ~same;
            ++n;
        }
        if (lane == 0) n_items = n;
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(ex.x, (uint32_t)((int64_t)ex.M * ex.ldx * 2));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(ex.y, (uint32_t)((int64_t)ex.M * ex.ldy * sizeof(TY)));
    const int t = lane & 15;
    for (int i = wave; i < n_items; i += kR1Waves) {
        const bool ok = t < item_n[i];
        expert_item<uint16_t, TY, true, NHT, true>(ex, lut, xr, yr, item_e[i], ok ? item_p[i][t] : 0, ok);
    }
    if (threadIdx.x == 0) *sync = 0u;  // no other workgroup of this launch reads it any more
}

// ------------------------------------------------------------------ experts backward
// Backward of FastMoEExperts.forward (moe.py:337-380: autograd of its three
// einsums, SiLU and the routing product, with the MoE STE of moe.py:289-294)
// over the routed (token, expert) pairs only -- a pair with routing weight
// zero adds nothing to dx or to the weight gradients -- in float32:
//   do = dout w;  g = Wg x, u = Wu x, s = silu(g), h = s u, o = Wd h
//   dw_pair = <dout, o>;  dh = Wd^T do;  dg = dh u silu'(g);  du = dh s
//   dx = Wg^T dg + Wu^T du;  dWg += dg x^T, dWu += du x^T, dWd += do h^T
// with W = code * gamma.  A workgroup takes a share of one expert's pairs
// (S workgroups per expert), two pairs at a time with 128 threads each
// (thread j owns hidden unit j), the expert's three matrices staged in LDS
// as float32 and the next pairs' rows prefetched during the current ones;
// each workgroup writes its weight-gradient sums, which
// moe_experts_bwd_reduce_kernel adds in workgroup order before the STE clamp.
constexpr int kEbSlots = 2;
constexpr int kEbH = 128;  // hidden units per expert <= 128
constexpr int kEbThreads = kEbSlots * kEbH;
struct ExpBwdArgs {
    const float *x;
    int64_t ldx;
    const float *dout;
    int64_t ldd;
    float *dx;
    int64_t ldgx;
    const int *list, *offset;  // pair ids t*k + j grouped by expert (walsh_moe_scatter)
    const float *topk_w;       // [M*k] routing weight of each pair
    int M, E, k, H, S;
    const uint8_t *pg, *pu, *pd;  // packed codes: gate / up [E][H][8], down [E][32][H/4]
    const float *gammas;          // [3]
    float *dpair;                 // [M*k] gradient of each pair's routing weight
    float *part;                  // [S][E][3][H*32] per-workgroup weight-gradient sums
};

__device__ __forceinline__ float packed_code(const uint8_t *row, int i) {
    const uint32_t b = row[i >> 2];
    return (float)((int)((b >> (6 - 2 * (i & 3))) & 3u) - 1);
}

__global__ __launch_bounds__(kEbThreads) void moe_experts_bwd_kernel(ExpBwdArgs a) {
    __shared__ float wg_l[kEbH][33], wu_l[kEbH][33], wd_l[32][kEbH + 1];
    __shared__ float xs[kEbSlots][32], os[kEbSlots][32], dos[kEbSlots][32];
    __shared__ float gs[kEbSlots][kEbH], us[kEbSlots][kEbH], hs[kEbSlots][kEbH];
    __shared__ float red[kEbSlots][2][32][2];
    const int e = (int)blockIdx.x / a.S, sp = (int)blockIdx.x % a.S;
    const int tid = threadIdx.x, slot = tid / kEbH, j = tid % kEbH;
    const int H = a.H, k = a.k;
    {
        const float g0 = a.gammas[0], g1 = a.gammas[1], g2 = a.gammas[2];
        for (int i = tid; i < H * 32; i += kEbThreads) {
            const int h = i >> 5, d = i & 31;
            wg_l[h][d] = packed_code(a.pg + ((int64_t)e * H + h) * 8, d) * g0;
            wu_l[h][d] = packed_code(a.pu + ((int64_t)e * H + h) * 8, d) * g1;
            wd_l[d][h] = packed_code(a.pd + ((int64_t)e * 32 + d) * (H / 4), h) * g2;
        }
    }
    const int p0 = a.offset[e], p1 = a.offset[e + 1];
    const int per = (p1 - p0 + a.S - 1) / a.S;
    const int b0 = p0 + sp * per, b1 = min(p1, b0 + per);
    const int iters = b1 > b0 ? (b1 - b0 + kEbSlots - 1) / kEbSlots : 0;
    float agw[32], auw[32], adw[32];
#pragma unroll
    for (int d = 0; d < 32; ++d) agw[d] = auw[d] = adw[d] = 0.f;
    // the slot's next pair: id, weight and (threads j < 32) element j of its
    // x and dout rows, loaded one iteration ahead
    int npid = -1;
    float nw = 0.f, nx = 0.f, nd = 0.f;
    auto fetch = [&](int it) {
        const int p = b0 + it * kEbSlots + slot;
        npid = (it < iters && p < b1) ? a.list[p] : -1;
        if (npid >= 0) {
            const int64_t t = npid / k;
            nw = a.topk_w[npid];
            if (j < 32) {
                nx = a.x[t * a.ldx + 32 * e + j];
                nd = a.dout[t * a.ldd + 32 * e + j];
            }
        }
    };
    fetch(0);
    for (int it = 0; it < iters; ++it) {
        const int pid = npid;
        const float w = nw;
        if (j < 32) {
            xs[slot][j] = nx;
            os[slot][j] = nd;
            dos[slot][j] = nd * w;
        }
        fetch(it + 1);
        __syncthreads();  // rows in LDS (and, on the first pass, the matrices)
        if (pid >= 0 && j < H) {
            float g = 0.f, u = 0.f, dh = 0.f;
#pragma unroll
            for (int d = 0; d < 32; ++d) {
                const float xv = xs[slot][d];
                g += wg_l[j][d] * xv;
                u += wu_l[j][d] * xv;
                dh += wd_l[d][j] * dos[slot][d];
            }
            const float sg = 1.0f / (1.0f + expf(-g));
            const float sv = g * sg, dsil = sg * (1.0f + g * (1.0f - sg));
            const float hv = sv * u, dg = dh * u * dsil, du = dh * sv;
#pragma unroll
            for (int d = 0; d < 32; ++d) {
                const float xv = xs[slot][d];
                agw[d] += dg * xv;
                auw[d] += du * xv;
                adw[d] += dos[slot][d] * hv;
            }
            gs[slot][j] = dg;
            us[slot][j] = du;
            hs[slot][j] = hv;
        }
        __syncthreads();
        {
            // thread (d = j % 32, q = j / 32) sums hidden units [32q, 32q + 32)
            const int d = j & 31, q = j >> 5;
            float vx = 0.f, vo = 0.f;
            if (pid >= 0) {
                const int h1 = min(H, 32 * q + 32);
                for (int h = 32 * q; h < h1; ++h) {
                    vx += gs[slot][h] * wg_l[h][d] + us[slot][h] * wu_l[h][d];
                    vo += hs[slot][h] * wd_l[d][h];
                }
            }
            vx += __shfl_xor(vx, 32, 64);  // q and q ^ 1 share a wave
            vo += __shfl_xor(vo, 32, 64);
            if ((j & 63) < 32) {
                red[slot][j >> 6][d][0] = vx;
                red[slot][j >> 6][d][1] = vo;
            }
        }
        __syncthreads();
        if (pid >= 0 && j < 32) {
            const float vx = red[slot][0][j][0] + red[slot][1][j][0];
            const float vo = red[slot][0][j][1] + red[slot][1][j][1];
            a.dx[(int64_t)(pid / k) * a.ldgx + 32 * e + j] = vx;
            float pw = os[slot][j] * vo;
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) pw += __shfl_xor(pw, off, 64);
            if (j == 0) a.dpair[pid] = pw;
        }
    }
    // the two slots' sums meet in LDS (the matrices are no longer needed)
    __syncthreads();
    if (slot == 1 && j < H) {
#pragma unroll
        for (int d = 0; d < 32; ++d) {
            wg_l[j][d] = agw[d];
            wu_l[j][d] = auw[d];
            wd_l[d][j] = adw[d];
        }
    }
    __syncthreads();
    if (slot == 0 && j < H) {
        float *dst = a.part + ((int64_t)sp * a.E + e) * 3 * H * 32;
#pragma unroll
        for (int d = 0; d < 32; ++d) {
            dst[j * 32 + d] = agw[d] + wg_l[j][d];
            dst[H * 32 + j * 32 + d] = auw[d] + wu_l[j][d];
            dst[2 * H * 32 + d * H + j] = adw[d] + wd_l[d][j];
        }
    }
}

// Weight gradients: the per-workgroup sums added in workgroup order, then
// clamp(., -2, 2) (the MoE STE); gate / up [E][H][32], down [E][32][H].
__global__ __launch_bounds__(256) void moe_experts_bwd_reduce_kernel(const float *__restrict__ part, int S, int E,
                                                                     int H, float *__restrict__ dg,
                                                                     float *__restrict__ du, float *__restrict__ dd) {
    const int64_t per = 3LL * H * 32, n = (int64_t)E * per;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int e = (int)(i / per), r = (int)(i % per);
        float v = 0.f;
        for (int sp = 0; sp < S; ++sp) v += part[((int64_t)sp * E + e) * per + r];
        v = fminf(fmaxf(v, -2.f), 2.f);
        const int kind = r / (H * 32), rr = r % (H * 32);
        float *dst = kind == 0 ? dg : (kind == 1 ? du : dd);
        if (dst) dst[(int64_t)e * H * 32 + rr] = v;
    }
}

static int experts_bwd_splits(int64_t E) {
    int64_t S = ceil_div(2 * (int64_t)device_info().cu_count, E);
    return (int)(S < 1 ? 1 : (S > 16 ? 16 : S));
}

static int route_out_check(const char *fn, int64_t M, int64_t E, int64_t k, const int *topk_idx, const float *topk_w,
                           const int *count, const float *probsum, int64_t n_part) {
    if (!count || !probsum || (M > 0 && (!topk_idx || !topk_w)))
        return set_error(WALSH_EINVAL, "%s: null output pointer", fn);
    if (n_part < 1 || n_part > 65536) return set_error(WALSH_EINVAL, "%s: n_part must be in [1, 65536]", fn);
    if (M < 0 || E < 1 || E > 16 * kMaxETiles || k < 1 || k > kMaxK || k > E)
        return set_error(WALSH_ENOTSUP, "%s: needs 1 <= k <= min(E, %d) and E <= %d (M=%lld E=%lld k=%lld)", fn, kMaxK,
                         16 * kMaxETiles, (long long)M, (long long)E, (long long)k);
    return WALSH_OK;
}

WALSH_EXPORT int walsh_moe_route_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, int64_t H1, const void *w1_frag,
                                     const void *w2_frag, int64_t E, int64_t k, float *probs, float *mask,
                                     float *weights_dense, int *topk_idx, float *topk_w, int *count, float *probsum,
                                     int64_t n_part, void *y, int64_t ldy, int dtype, int ydtype, void *stream) {
    const char *fn = "walsh_moe_route_fwd";
    int rc = route_out_check(fn, M, E, k, topk_idx, topk_w, count, probsum, n_part);
    if (rc) return rc;
    if ((M > 0 && !x) || !w1_frag || !w2_frag) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
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
    if (M == 0) {
        launch(moe_zero_kernel, dim3(1), dim3(256), 0, s, count, probsum, (int)(n_part * E));
        return check_hip(hipGetLastError(), fn);
    }
    RouterArgs a;
    a.x = x;
    a.ldx = ldx;
    a.C = (int)C;
    a.H1 = (int)H1;
    a.w1f = w1_frag;
    a.w2f = w2_frag;
    a.net = (int)ceil_div(E, 16);
    a.o = RouteOut{(int)M,   (int)E,  (int)k,   probs, mask, weights_dense,        topk_idx,
                   topk_w,   count,   probsum,  (int)n_part, y, ldy, ydtype == WALSH_BF16};
    const dim3 G(grid_cap(ceil_div(M, 16), n_part)), B(kMoeThreads);
#define WALSH_ROUTE(NE)                                                                               \
    if (dtype == WALSH_BF16) launch((moe_route_kernel<uint16_t, true, NE>), G, B, 0, s, a); \
    else launch((moe_route_kernel<float, false, NE>), G, B, 0, s, a);
    if (a.net <= 1) { WALSH_ROUTE(1) } else if (a.net <= 2) { WALSH_ROUTE(2) } else { WALSH_ROUTE(4) }
#undef WALSH_ROUTE
    return check_hip(hipGetLastError(), fn);
}

// workspace: h [M][H] bf16, then (M <= kR1SmallRows) the partial logits
// [H/16][M][E] float
static int64_t router_h_bytes(int64_t M, int64_t H) { return ceil_div(M * H * 2, 256) * 256; }

WALSH_EXPORT int64_t walsh_moe_router_wide_workspace_bytes(int64_t M, int64_t H, int64_t E) {
    if (M < 0 || H <= 0 || E <= 0) return 0;
    return router_h_bytes(M, H) + (M <= kR1SmallRows ? (H / 16) * M * E * 4 : 0);
}

WALSH_EXPORT int walsh_moe_router_wide_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, int64_t H,
                                           const void *w1, const void *w2, int64_t E, int64_t k, void *work,
                                           int64_t work_bytes, float *probs, float *mask, float *weights_dense,
                                           int *topk_idx, float *topk_w, int *count, float *probsum, int64_t n_part,
                                           void *y, int64_t ldy, int ydtype, void *stream) {
    const char *fn = "walsh_moe_router_wide_fwd";
    int rc = route_out_check(fn, M, E, k, topk_idx, topk_w, count, probsum, n_part);
    if (rc) return rc;
    if ((M > 0 && (!x || !work)) || !w1 || !w2) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (C % (32 * kR1Waves) || H % 128 || H > kR2MaxH || E % 4 || ldx < C || (y && ldy < 32 * E))
        return set_error(WALSH_ENOTSUP, "%s: needs C %% %d == 0, H %% 128 == 0, H <= %d, E %% 4 == 0 (C=%lld H=%lld "
                         "E=%lld)", fn, 32 * kR1Waves, kR2MaxH, (long long)C, (long long)H, (long long)E);
    if (work_bytes < walsh_moe_router_wide_workspace_bytes(M, H, E))
        return set_error(WALSH_EINVAL, "%s: workspace of %lld bytes, needs %lld", fn, (long long)work_bytes,
                         (long long)walsh_moe_router_wide_workspace_bytes(M, H, E));
    if (ydtype != WALSH_F32 && ydtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: ydtype", fn);
    const int64_t ysz = ydtype == WALSH_BF16 ? 2 : 4;
    if (ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)work % 256 || (uintptr_t)w1 % 16 || (uintptr_t)w2 % 16 ||
        (y && ((uintptr_t)y % 16 || ldy % (16 / ysz))))
        return set_error(WALSH_ENOTSUP, "%s: operands and rows must be 16-byte aligned (workspace 256)", fn);
    if (M * ldx * 2 > (int64_t)kMaxBufferBytes || M * H * 2 > (int64_t)kMaxBufferBytes ||
        H * C * 2 > (int64_t)kMaxBufferBytes)
        return set_error(WALSH_ENOTSUP, "%s: operands above 2^31 bytes", fn);
    if (router_w2_lds_bytes((int)H, 4) + 8 * kMaxE > (size_t)device_info().max_shared_per_block)
        return set_error(WALSH_ENOTSUP, "%s: H=%lld needs more LDS than a workgroup has", fn, (long long)H);
    hipStream_t s = (hipStream_t)stream;
    if (M == 0) {
        launch(moe_zero_kernel, dim3(1), dim3(256), 0, s, count, probsum, (int)(n_part * E));
        return check_hip(hipGetLastError(), fn);
    }
    uint16_t *h = (uint16_t *)work;
    const RouteOut o{(int)M, (int)E, (int)k, probs, mask, weights_dense, topk_idx, topk_w, count, probsum,
                     (int)n_part, y, ldy, ydtype == WALSH_BF16};
    if (M <= kR1SmallRows) {
        float *lpart = (float *)((char *)work + router_h_bytes(M, H));
        launch(router_w1_small_kernel, dim3((unsigned)(H / 16), (unsigned)ceil_div(M, 16)), dim3(64 * kR1Waves), 0, s,
               (const uint16_t *)x, ldx, (int)M, (int)C, (const uint16_t *)w1, h, H, (const uint16_t *)w2, (int)E,
               lpart);
        rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
        launch(router_topk_part_kernel, dim3((unsigned)(M < n_part ? M : n_part)), dim3(kMoeThreads), 0, s,
               (const float *)lpart, (int)(H / 16), o);
        return check_hip(hipGetLastError(), fn);
    }
    Gemm256Args g{};
    g.x = x;
    g.ldx = ldx;
    g.M = (int)M;
    g.N = (int)H;
    g.K = (int)C;
    g.Kp = (int)C;
    g.B = w1;
    g.beta = nullptr;
    g.out_o = (int)H;
    g.y = h;
    g.ldy = H;
    gemm256_launch<kEpiSilu>(g, s);
    rc = check_hip(hipGetLastError(), fn);
    if (rc) return rc;
    const int64_t tiles = ceil_div(M, 64), grid = tiles < n_part ? tiles : n_part;
    launch(router_w2_topk_kernel<4>, dim3((unsigned)grid), dim3(64 * kR2Waves), (uint32_t)router_w2_lds_bytes((int)H, 4),
           s, (const uint16_t *)h, (int64_t)H, (int)H, (const uint16_t *)w2, o);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int64_t walsh_moe_decode_workspace_bytes(int64_t M, int64_t H, int64_t E) {
    if (M < 1 || M > kDecTok || H <= 0 || E <= 0) return 0;
    return router_h_bytes(M, H) + (H / 16) * M * E * 4;
}

WALSH_EXPORT int walsh_moe_decode_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, int64_t H, const void *w1,
                                      const void *w2, int64_t E, int64_t k, int64_t He, const uint8_t *gate_frag,
                                      const uint8_t *up_frag, const uint8_t *down_frag, const float *gammas,
                                      void *work, int64_t work_bytes, unsigned *sync, float *probs, float *mask,
                                      float *weights_dense, int *topk_idx, float *topk_w, int *count,
                                      float *probsum, int64_t n_part, void *y, int64_t ldy, int ydtype,
                                      void *stream) {
    const char *fn = "walsh_moe_decode_fwd";
    int rc = route_out_check(fn, M, E, k, topk_idx, topk_w, count, probsum, n_part);
    if (rc) return rc;
    if (!x || !w1 || !w2 || !gate_frag || !up_frag || !down_frag || !gammas || !work || !sync || !y)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 1 || M > kDecTok)
        return set_error(WALSH_ENOTSUP, "%s: takes 1..%d tokens (M=%lld)", fn, kDecTok, (long long)M);
    // the routing workgroup writes partial row t of count / probsum for token t
    if (n_part < M)
        return set_error(WALSH_EINVAL, "%s: n_part=%lld partial rows for M=%lld tokens (one row per token)", fn,
                         (long long)n_part, (long long)M);
    if (C % (32 * kR1Waves) || H % 128 || H > kR2MaxH || E % 4 || C != 32 * E || ldx < C || ldy < 32 * E)
        return set_error(WALSH_ENOTSUP, "%s: needs C %% %d == 0, H %% 128 == 0, H <= %d, E %% 4 == 0, C == 32 E "
                         "(C=%lld H=%lld E=%lld)", fn, 32 * kR1Waves, kR2MaxH, (long long)C, (long long)H,
                         (long long)E);
    if (He != 64 && He != 128 && He != 256)
        return set_error(WALSH_ENOTSUP, "%s: expert hidden must be 64, 128 or 256", fn);
    if (work_bytes < walsh_moe_decode_workspace_bytes(M, H, E))
        return set_error(WALSH_EINVAL, "%s: workspace of %lld bytes, needs %lld", fn, (long long)work_bytes,
                         (long long)walsh_moe_decode_workspace_bytes(M, H, E));
    if (ydtype != WALSH_F32 && ydtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: ydtype", fn);
    const int64_t ysz = ydtype == WALSH_BF16 ? 2 : 4;
    if (ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)work % 256 || (uintptr_t)w1 % 16 || (uintptr_t)w2 % 16 ||
        (uintptr_t)y % 16 || ldy % (16 / ysz) || (uintptr_t)sync % 4)
        return set_error(WALSH_ENOTSUP, "%s: operands and rows must be 16-byte aligned (workspace 256)", fn);
    if (H * C * 2 > (int64_t)kMaxBufferBytes) return set_error(WALSH_ENOTSUP, "%s: W1 above 2^31 bytes", fn);
    uint16_t *h = (uint16_t *)work;
    float *lpart = (float *)((char *)work + router_h_bytes(M, H));
    const RouteOut o{(int)M, (int)E, (int)k, probs, mask, weights_dense, topk_idx, topk_w, count, probsum,
                     (int)n_part, y, ldy, ydtype == WALSH_BF16};
    ExpArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.y = y;
    a.ldy = ldy;
    a.M = (int)M;
    a.E = (int)E;
    a.k = (int)k;
    a.H = (int)He;
    a.gate_f = gate_frag;
    a.up_f = up_frag;
    a.down_f = down_frag;
    a.gammas = gammas;
    a.topk_w = topk_w;
    const dim3 G((unsigned)(H / 16)), B(64 * kR1Waves);
    hipStream_t s = (hipStream_t)stream;
#define WALSH_DEC_LAUNCH(NH)                                                                                      \
    if (ydtype == WALSH_BF16)                                                                                     \
        launch((moe_decode_kernel<uint16_t, NH>), G, B, 0, s, (const uint16_t *)x, ldx, (int)C,                 \
               (const uint16_t *)w1, h, (const uint16_t *)w2, lpart, o, a, sync);                                 \
    else                                                                                                          \
        launch((moe_decode_kernel<float, NH>), G, B, 0, s, (const uint16_t *)x, ldx, (int)C, (const uint16_t *)w1, \
               h, (const uint16_t *)w2, lpart, o, a, sync);
    if (He == 64) { WALSH_DEC_LAUNCH(4) }
    else if (He == 128) { WALSH_DEC_LAUNCH(8) }
    else { WALSH_DEC_LAUNCH(16) }
#undef WALSH_DEC_LAUNCH
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int64_t walsh_moe_experts_bwd_workspace_bytes(int64_t E, int64_t H) {
    if (E < 1 || E > kMaxE || H < 16 || H > kEbH) return 0;
    return (int64_t)experts_bwd_splits(E) * E * 3 * H * 32 * 4;
}

WALSH_EXPORT int walsh_moe_experts_bwd(const float *x, int64_t ldx, const float *dout, int64_t ldd, int64_t M,
                                       int64_t E, int64_t k, int64_t H, const uint8_t *gate_packed,
                                       const uint8_t *up_packed, const uint8_t *down_packed, const float *gammas,
                                       const int *list, const int *offset, const float *topk_w, float *dx,
                                       int64_t ldgx, float *d_pair_w, float *dgate, float *dup, float *ddown,
                                       void *work, int64_t work_bytes, void *stream) {
    const char *fn = "walsh_moe_experts_bwd";
    if (!gate_packed || !up_packed || !down_packed || !gammas || !offset || !work ||
        (M > 0 && (!x || !dout || !list || !topk_w || !dx || !d_pair_w)))
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || E < 1 || E > kMaxE || k < 1 || k > E || H < 16 || H > kEbH || H % 16 || ldx < 32 * E ||
        ldd < 32 * E || ldgx < 32 * E)
        return set_error(WALSH_ENOTSUP, "%s: needs E <= %d, hidden H in [16, %d] (multiple of 16), rows >= 32 E", fn,
                         kMaxE, kEbH);
    if (work_bytes < walsh_moe_experts_bwd_workspace_bytes(E, H))
        return set_error(WALSH_EINVAL, "%s: workspace of %lld bytes, needs %lld", fn, (long long)work_bytes,
                         (long long)walsh_moe_experts_bwd_workspace_bytes(E, H));
    hipStream_t s = (hipStream_t)stream;
    const int S = experts_bwd_splits(E);
    ExpBwdArgs a;
    a.x = x;
    a.ldx = ldx;
    a.dout = dout;
    a.ldd = ldd;
    a.dx = dx;
    a.ldgx = ldgx;
    a.list = list;
    a.offset = offset;
    a.topk_w = topk_w;
    a.M = (int)M;
    a.E = (int)E;
    a.k = (int)k;
    a.H = (int)H;
    a.S = S;
    a.pg = gate_packed;
    a.pu = up_packed;
    a.pd = down_packed;
    a.gammas = gammas;
    a.dpair = d_pair_w;
    a.part = (float *)work;
    launch(moe_experts_bwd_kernel, dim3((unsigned)(E * S)), dim3(kEbThreads), 0, s, a);
    int rc = check_hip(hipGetLastError(), fn);
    if (rc) return rc;
    int64_t grid = ceil_div(E * 3 * H * 32, 256);
    if (grid > 4096) grid = 4096;
    launch(moe_experts_bwd_reduce_kernel, dim3((unsigned)grid), dim3(256), 0, s, (const float *)work, S, (int)E,
           (int)H, dgate, dup, ddown);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_moe_topk_fwd(const float *logits, int64_t M, int64_t E, int64_t k, float *probs, float *mask,
                                    float *weights_dense, int *topk_idx, float *topk_w, int *count, float *probsum,
                                    int64_t n_part, void *stream) {
    const char *fn = "walsh_moe_topk_fwd";
    int rc = route_out_check(fn, M, E, k, topk_idx, topk_w, count, probsum, n_part);
    if (rc) return rc;
    if (M > 0 && !logits) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    hipStream_t s = (hipStream_t)stream;
    if (M == 0) {
        launch(moe_zero_kernel, dim3(1), dim3(256), 0, s, count, probsum, (int)(n_part * E));
        return check_hip(hipGetLastError(), fn);
    }
    RouteOut o{(int)M, (int)E, (int)k, probs, mask, weights_dense, topk_idx, topk_w, count, probsum, (int)n_part,
               nullptr, 0, 0};
    const int net = (int)ceil_div(E, 16);
    if (net <= 1) {
        const dim3 G(grid_cap(ceil_div(M, 16), n_part)), B(kMoeThreads);
        launch(moe_topk_kernel<1>, G, B, 0, s, logits, net, o);
    } else {
        // one wavefront per token
        const dim3 G(grid_cap(M, n_part)), B(kMoeThreads);
        launch(moe_topk_rank_kernel, G, B, 0, s, logits, o);
    }
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_moe_scatter(const int *topk_idx, int64_t M, int64_t E, int64_t k, const int *count_part,
                                   const float *probsum_part, int64_t n_part, int *count, float *probsum, int *cursor,
                                   int *list, int *offset, int *tile_off, void *stream) {
    const char *fn = "walsh_moe_scatter";
    if ((M > 0 && (!topk_idx || !list)) || !count_part || !probsum_part || !count || !probsum || !cursor ||
        !offset || !tile_off)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || E < 1 || E > kMaxE || k < 1 || n_part < 1 || n_part > 65536)
        return set_error(WALSH_EINVAL, "%s: bad shape (M=%lld E=%lld k=%lld n_part=%lld)", fn, (long long)M,
                         (long long)E, (long long)k, (long long)n_part);
    hipStream_t s = (hipStream_t)stream;
    const int64_t n_pairs = M * k;
    if (n_pairs <= kScatterSmallPairs) {
        launch(moe_scatter_small_kernel, dim3(1), dim3(kMaxE * kFinSlices), 0, s, topk_idx, (int)n_pairs,
               count_part, probsum_part, (int)n_part, (int)E, count, probsum, cursor, offset, tile_off, list);
        return check_hip(hipGetLastError(), fn);
    }
    launch(moe_finalize_kernel, dim3(1), dim3(kMaxE * kFinSlices), 0, s, count_part, probsum_part, (int)n_part,
                       (int)E, count, probsum, cursor, offset, tile_off);
    if (n_pairs > 0) {
        const int64_t grid = ceil_div(n_pairs, 256 * kScatterPerThread);
        launch(moe_scatter_kernel, dim3((unsigned)grid), dim3(256), 0, s, topk_idx, n_pairs, (int)E,
                           offset, cursor, list);
    }
    return check_hip(hipGetLastError(), fn);
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
    if (dtype == WALSH_F32) launch((moe_experts_kernel<float, float, false, NH>), G, B, 0, s, a);  \
    else if (ydtype == WALSH_BF16)                                                                            \
        launch((moe_experts_kernel<uint16_t, uint16_t, true, NH>), G, B, 0, s, a);                \
    else launch((moe_experts_kernel<uint16_t, float, true, NH>), G, B, 0, s, a);
    if (H == 64) { WALSH_EXP_LAUNCH(4) } else if (H == 128) { WALSH_EXP_LAUNCH(8) } else { WALSH_EXP_LAUNCH(16) }
#undef WALSH_EXP_LAUNCH
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_moe_ffn_fwd(const void *x, int64_t ldx, int64_t M, int64_t C, const void *w1_frag,
                                   const void *w2_frag, int64_t E, int64_t k, int64_t H, const uint16_t *gate_frag,
                                   const uint16_t *up_frag, const uint16_t *down_frag, const float *gammas,
                                   int *topk_idx, float *topk_w, int *count, float *probsum, int64_t n_part,
                                   void *y, int64_t ldy, int dtype, int ydtype, void *stream) {
    const char *fn = "walsh_moe_ffn_fwd";
    if (!w1_frag || !w2_frag || !gate_frag || !up_frag || !down_frag || !gammas || !count || !probsum ||
        (M > 0 && (!x || !y || !topk_idx || !topk_w)))
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (C != kFfnC || E != kFfnE || dtype != WALSH_BF16 || (H != 64 && H != 128) || k < 1 || k > kMaxK || M < 0 ||
        (ydtype != WALSH_F32 && ydtype != WALSH_BF16))
        return set_error(WALSH_ENOTSUP, "%s: needs bf16 input, n_embd 512 (16 experts), hidden 64/128, k <= 8", fn);
    const int64_t ysz = ydtype == WALSH_BF16 ? 2 : 4;
    if (ldx < C || ldy < C || ldx % 8 || ldy % (16 / ysz) || (uintptr_t)x % 16 || (uintptr_t)y % 16)
        return set_error(WALSH_ENOTSUP, "%s: x and y rows must be 16-byte aligned", fn);
    if (M * ldx * 2 > (int64_t)kMaxBufferBytes) return set_error(WALSH_ENOTSUP, "%s: input too large", fn);
    if (n_part < 1 || n_part > 65536) return set_error(WALSH_EINVAL, "%s: n_part must be in [1, 65536]", fn);
    hipStream_t s = (hipStream_t)stream;
    if (M == 0) {
        launch(moe_zero_kernel, dim3(1), dim3(256), 0, s, count, probsum, (int)(n_part * E));
        return check_hip(hipGetLastError(), fn);
    }
    FfnArgs a;
    a.x = (const uint16_t *)x;
    a.ldx = ldx;
    a.M = (int)M;
    a.k = (int)k;
    a.w1f = (const uint4 *)w1_frag;
    a.w2f = (const uint2 *)w2_frag;
    a.gate_f = gate_frag;
    a.up_f = up_frag;
    a.down_f = down_frag;
    a.gammas = gammas;
    a.topk_idx = topk_idx;
    a.topk_w = topk_w;
    a.count = count;
    a.probsum = probsum;
    a.n_part = (int)n_part;
    a.y = y;
    a.ldy = ldy;
    int64_t g = ceil_div(M, kFfnTok);
    const int64_t cap = device_info().cu_count;
    if (g > cap) g = cap;
    if (g > n_part) g = n_part;
    const dim3 G((unsigned)g), B(kFfnThreads);
#define WALSH_FFN(NHV)                                                                 \
    if (ydtype == WALSH_F32) launch((moe_ffn_kernel<float, NHV>), G, B, 0, s, a); \
    else launch((moe_ffn_kernel<uint16_t, NHV>), G, B, 0, s, a);
    if (H == 64) { WALSH_FFN(4) } else { WALSH_FFN(8) }
#undef WALSH_FFN
    return check_hip(hipGetLastError(), fn);
}
