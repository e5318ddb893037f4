// mHC (manifold hyper-connection) residual-stream kernels.
//
//   walsh_sinkhorn_fwd  SinkhornKnopp.forward (src/model/mhc.py:214-229)
//   walsh_mhc_pre_fwd   the three ResidualStreamMapping.forward calls of one
//                       mHCResidualStream.forward plus its H_pre @ x
//                       (mhc.py:283-318, 345-364), fused: one pass over x
//   walsh_mhc_post_fwd  x_new = H_res @ x + H_post^T (x) out (mhc.py:366-381)
//
// Stream tensors are [M tokens][n streams][C] (row stride ldx >= n*C).
#include <type_traits>

#include "common.h"

namespace walsh {

constexpr int kMaxStreams = 4;            // n*n + 2n <= 24 outputs -> 2 MMA tiles
constexpr int kPhiRows = 32;              // projection rows padded to 2 x 16
constexpr int kPreTok = 32;               // tokens per workgroup (2 x 16)
constexpr int kPreWaves = 4;              // K split across 4 wavefronts
constexpr int kPreThreads = 64 * kPreWaves;

// Sinkhorn-Knopp on an n x n matrix in registers: M = exp(H); n_iter x
// {divide each column by (its sum + eps); divide each row by (its sum + eps)}.
template <int NMAX>
__device__ __forceinline__ void sinkhorn_regs(float (&m)[NMAX][NMAX], int n, int n_iter, float eps) {
#pragma unroll
    for (int i = 0; i < NMAX; ++i)
#pragma unroll
        for (int j = 0; j < NMAX; ++j) m[i][j] = (i < n && j < n) ? expf(m[i][j]) : 0.f;
    for (int it = 0; it < n_iter; ++it) {
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
            if (j >= n) continue;
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) s += (i < n) ? m[i][j] : 0.f;
            const float d = s + eps;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) m[i][j] = __fdiv_rn(m[i][j], d);
        }
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
            if (i >= n) continue;
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < NMAX; ++j) s += (j < n) ? m[i][j] : 0.f;
            const float d = s + eps;
#pragma unroll
            for (int j = 0; j < NMAX; ++j) m[i][j] = __fdiv_rn(m[i][j], d);
        }
    }
}

__device__ __forceinline__ float sigmoidf(float v) { return __fdiv_rn(1.0f, 1.0f + expf(-v)); }

// Sum over the 4 lanes of a quad with DPP quad_perm moves (no LDS round trip).
__device__ __forceinline__ float quad_sum(float v) {
    const int x1 = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true);    // lanes ^1
    const float s = v + __int_as_float(x1);
    const int x2 = __builtin_amdgcn_mov_dpp(__float_as_int(s), 0x4E, 0xF, 0xF, true);    // lanes ^2
    return s + __int_as_float(x2);
}

// Per-token constraints with 4 lanes per token (lane r = row r of the n x n
// residual matrix; r < n active).  dynf(o) returns the RMS-scaled projection
// output o of this token.  Column sums of the Sinkhorn iteration are quad
// shuffles; each lane divides its own row, so a whole wavefront projects 16
// tokens at once.  Results go to hpre_lds[t*4 + r] and (if tok valid) global.
// In two parts: the gates (H_pre, H_post and exp of the residual logits),
// then the Sinkhorn iterations and the stores, so that a caller can publish
// H_pre before running the iterations.
struct QuadGates {
    float pre, post;
    float m[kMaxStreams];
};

template <typename DynF>
__device__ __forceinline__ QuadGates token_gates_quad(int r, int n, const float *coef, const float *bias, DynF dynf) {
    const bool act = r < n;
    QuadGates q;
    q.pre = 0.f;
    q.post = 0.f;
    if (act) {
        q.pre = __builtin_amdgcn_rcpf(1.0f + __expf(-(coef[0] * dynf(r) + bias[r])));
        q.post = 2.0f * __builtin_amdgcn_rcpf(1.0f + __expf(-(coef[1] * dynf(n + r) + bias[n + r])));
    }
#pragma unroll
    for (int j = 0; j < kMaxStreams; ++j)
        q.m[j] = (act && j < n) ? __expf(coef[2] * dynf(2 * n + r * n + j) + bias[2 * n + r * n + j]) : 0.f;
    return q;
}

// One Sinkhorn iteration on a quad: column sums by quad shuffles, then the
// lane's own row.
__device__ __forceinline__ void sinkhorn_quad_step(float (&m)[kMaxStreams], int n, float sk_eps) {
#pragma unroll
    for (int j = 0; j < kMaxStreams; ++j) {
        const float cs = quad_sum(m[j]);
        if (j < n) m[j] *= __builtin_amdgcn_rcpf(cs + sk_eps);
    }
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxStreams; ++j) rs += (j < n) ? m[j] : 0.f;
    const float rd = __builtin_amdgcn_rcpf(rs + sk_eps);
#pragma unroll
    for (int j = 0; j < kMaxStreams; ++j)
        if (j < n) m[j] *= rd;
}

__device__ __forceinline__ void token_store_quad(const QuadGates &q, int r, int tok, int M, int n, float *h_pre,
                                                 float *h_post, float *h_res) {
    if (r < n && tok < M) {
        h_pre[(int64_t)tok * n + r] = q.pre;
        h_post[(int64_t)tok * n + r] = q.post;
#pragma unroll
        for (int j = 0; j < kMaxStreams; ++j)
            if (j < n) h_res[((int64_t)tok * n + r) * n + j] = q.m[j];
    }
}

__device__ __forceinline__ void token_sinkhorn_quad(QuadGates &q, int r, int tok, int M, int n, int n_iter,
                                                    float sk_eps, float *h_pre, float *h_post, float *h_res) {
    for (int it = 0; it < n_iter; ++it) sinkhorn_quad_step(q.m, n, sk_eps);
    token_store_quad(q, r, tok, M, n, h_pre, h_post, h_res);
}

// v of quad lane S, broadcast to the quad (DPP quad_perm [S, S, S, S]).
template <int S>
__device__ __forceinline__ float quad_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), S * 0x55, 0xF, 0xF, true));
}

template <typename DynF>
__device__ __forceinline__ void token_constraints_quad(int t, int r, int tok, int M, int n, const float *coef,
                                                       const float *bias, int n_iter, float sk_eps, DynF dynf,
                                                       float *hpre_lds, float *h_pre, float *h_post, float *h_res) {
    QuadGates q = token_gates_quad(r, n, coef, bias, dynf);
    hpre_lds[t * 4 + r] = q.pre;
    token_sinkhorn_quad(q, r, tok, M, n, n_iter, sk_eps, h_pre, h_post, h_res);
}

// ---------------------------------------------------------------- sinkhorn
// Backward of sinkhorn_regs for the output gradient g (the autograd of
// SinkhornKnopp.forward, src/model/mhc.py:214-229, which the reference leaves
// to torch): per matrix, walking the iterations backwards, the state S_k
// before iteration k is recomputed from exp(h) with the forward's own
// operations (so every intermediate is bit-identical to the forward's), then
//   row step    U = T / r,  r_i = sum_j T_ij + eps:  dT_ij = (G_ij - sum_j' G_ij' U_ij') / r_i
//   column step T = S / c,  c_j = sum_i S_ij + eps:  dS_ij = (dT_ij - sum_i' dT_i'j T_i'j) / c_j
// and finally dh = G .* exp(h).  O(n_iter^2) small iterations per matrix.
template <int NMAX>
__global__ void sinkhorn_bwd_kernel(const float *__restrict__ h, const float *__restrict__ g, int64_t batch, int n,
                                    int n_iter, float eps, float *__restrict__ dh) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < batch; b += (int64_t)gridDim.x * blockDim.x) {
        float m0[NMAX][NMAX], G[NMAX][NMAX];
        const float *src = h + b * n * n;
        const float *gs = g + b * n * n;
#pragma unroll
        for (int i = 0; i < NMAX; ++i)
#pragma unroll
            for (int j = 0; j < NMAX; ++j) {
                m0[i][j] = (i < n && j < n) ? expf(src[i * n + j]) : 0.f;
                G[i][j] = (i < n && j < n) ? gs[i * n + j] : 0.f;
            }
        for (int k = n_iter - 1; k >= 0; --k) {
            float S[NMAX][NMAX], T[NMAX][NMAX], c[NMAX], r[NMAX];
#pragma unroll
            for (int i = 0; i < NMAX; ++i)
#pragma unroll
                for (int j = 0; j < NMAX; ++j) S[i][j] = m0[i][j];
            for (int it = 0; it <= k; ++it) {
#pragma unroll
                for (int j = 0; j < NMAX; ++j) {
                    float sum = 0.f;
#pragma unroll
                    for (int i = 0; i < NMAX; ++i) sum += (i < n) ? S[i][j] : 0.f;
                    c[j] = sum + eps;
#pragma unroll
                    for (int i = 0; i < NMAX; ++i) T[i][j] = (j < n) ? __fdiv_rn(S[i][j], c[j]) : 0.f;
                }
#pragma unroll
                for (int i = 0; i < NMAX; ++i) {
                    float sum = 0.f;
#pragma unroll
                    for (int j = 0; j < NMAX; ++j) sum += (j < n) ? T[i][j] : 0.f;
                    r[i] = sum + eps;
                    if (it < k) {
#pragma unroll
                        for (int j = 0; j < NMAX; ++j) S[i][j] = (i < n) ? __fdiv_rn(T[i][j], r[i]) : 0.f;
                    }
                }
            }
            // now T, c, r are iteration k's; U = T / r
            float dT[NMAX][NMAX];
#pragma unroll
            for (int i = 0; i < NMAX; ++i) {
                float dot = 0.f;
#pragma unroll
                for (int j = 0; j < NMAX; ++j) dot += (i < n && j < n) ? G[i][j] * __fdiv_rn(T[i][j], r[i]) : 0.f;
#pragma unroll
                for (int j = 0; j < NMAX; ++j) dT[i][j] = (i < n && j < n) ? __fdiv_rn(G[i][j] - dot, r[i]) : 0.f;
            }
#pragma unroll
            for (int j = 0; j < NMAX; ++j) {
                float dot = 0.f;
#pragma unroll
                for (int i = 0; i < NMAX; ++i) dot += (i < n && j < n) ? dT[i][j] * T[i][j] : 0.f;
#pragma unroll
                for (int i = 0; i < NMAX; ++i) G[i][j] = (i < n && j < n) ? __fdiv_rn(dT[i][j] - dot, c[j]) : 0.f;
            }
        }
        float *dst = dh + b * n * n;
#pragma unroll
        for (int i = 0; i < NMAX; ++i)
#pragma unroll
            for (int j = 0; j < NMAX; ++j)
                if (i < n && j < n) dst[i * n + j] = G[i][j] * m0[i][j];
    }
}

// The same gradient with the states S_k kept in LDS (one column per thread,
// [n_iter][NMAX*NMAX][threads]): one forward sweep stores them, one backward
// sweep reads them, O(n_iter) per matrix.  Used when the states fit.
constexpr int kSkBwdThreads = 64;
template <int NMAX>
__global__ __launch_bounds__(kSkBwdThreads) void sinkhorn_bwd_lds_kernel(const float *__restrict__ h,
                                                                         const float *__restrict__ g, int64_t batch,
                                                                         int n, int n_iter, float eps,
                                                                         float *__restrict__ dh) {
    extern __shared__ float st[];
    const int tid = threadIdx.x;
    const int64_t b = (int64_t)blockIdx.x * kSkBwdThreads + tid;
    if (b >= batch) return;  // no barrier: each thread uses only its own LDS column
    auto at = [&](int k, int e) -> float & { return st[((int64_t)k * NMAX * NMAX + e) * kSkBwdThreads + tid]; };
    float m0[NMAX][NMAX], S[NMAX][NMAX];
    const float *src = h + b * n * n;
#pragma unroll
    for (int i = 0; i < NMAX; ++i)
#pragma unroll
        for (int j = 0; j < NMAX; ++j) S[i][j] = m0[i][j] = (i < n && j < n) ? expf(src[i * n + j]) : 0.f;
    for (int k = 0; k < n_iter; ++k) {
#pragma unroll
        for (int i = 0; i < NMAX; ++i)
#pragma unroll
            for (int j = 0; j < NMAX; ++j) at(k, i * NMAX + j) = S[i][j];
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) sum += (i < n) ? S[i][j] : 0.f;
            const float c = sum + eps;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) S[i][j] = (j < n) ? __fdiv_rn(S[i][j], c) : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < NMAX; ++j) sum += (j < n) ? S[i][j] : 0.f;
            const float r = sum + eps;
#pragma unroll
            for (int j = 0; j < NMAX; ++j) S[i][j] = (i < n) ? __fdiv_rn(S[i][j], r) : 0.f;
        }
    }
    float G[NMAX][NMAX];
    const float *gs = g + b * n * n;
#pragma unroll
    for (int i = 0; i < NMAX; ++i)
#pragma unroll
        for (int j = 0; j < NMAX; ++j) G[i][j] = (i < n && j < n) ? gs[i * n + j] : 0.f;
    for (int k = n_iter - 1; k >= 0; --k) {
        float T[NMAX][NMAX], c[NMAX], r[NMAX];
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) sum += (i < n) ? at(k, i * NMAX + j) : 0.f;
            c[j] = sum + eps;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) T[i][j] = (j < n) ? __fdiv_rn(at(k, i * NMAX + j), c[j]) : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < NMAX; ++j) sum += (j < n) ? T[i][j] : 0.f;
            r[i] = sum + eps;
        }
        float dT[NMAX][NMAX];
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
            float dot = 0.f;
#pragma unroll
            for (int j = 0; j < NMAX; ++j) dot += (i < n && j < n) ? G[i][j] * __fdiv_rn(T[i][j], r[i]) : 0.f;
#pragma unroll
            for (int j = 0; j < NMAX; ++j) dT[i][j] = (i < n && j < n) ? __fdiv_rn(G[i][j] - dot, r[i]) : 0.f;
        }
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) dot += (i < n && j < n) ? dT[i][j] * T[i][j] : 0.f;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) G[i][j] = (i < n && j < n) ? __fdiv_rn(dT[i][j] - dot, c[j]) : 0.f;
        }
    }
    float *dst = dh + b * n * n;
#pragma unroll
    for (int i = 0; i < NMAX; ++i)
#pragma unroll
        for (int j = 0; j < NMAX; ++j)
            if (i < n && j < n) dst[i * n + j] = G[i][j] * m0[i][j];
}

// ---------------------------------------------------------------- stream mixing for training
// Dense rows: x / dx / dnew [M][n][C], li / dli / out / dout [M][C] (one
// dtype T), h_pre / h_post [M][n], h_res [M][n][n] float32.  One wavefront
// per token; lane l covers columns 4l + 256k; sums over the C columns are
// per-lane partials reduced across the wavefront with xor shuffles.
constexpr int kMixWaves = 4;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <typename T>
__global__ __launch_bounds__(64 * kMixWaves) void mhc_agg_fwd_kernel(const T *__restrict__ x,
                                                                     const float *__restrict__ h_pre,
                                                                     T *__restrict__ li, int64_t M, int n, int C) {
    const int lane = threadIdx.x & 63;
    for (int64_t t = (int64_t)blockIdx.x * kMixWaves + (threadIdx.x >> 6); t < M; t += (int64_t)gridDim.x * kMixWaves) {
        float hp[kMaxStreams];
#pragma unroll
        for (int s = 0; s < kMaxStreams; ++s) hp[s] = s < n ? h_pre[t * n + s] : 0.f;
        for (int c = 4 * lane; c < C; c += 256) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < kMaxStreams; ++s)
                if (s < n) acc += hp[s] * load4(x + (t * n + s) * C + c);
            store4(li + t * C + c, acc);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(64 * kMixWaves) void mhc_agg_bwd_kernel(const T *__restrict__ x,
                                                                     const float *__restrict__ h_pre,
                                                                     const T *__restrict__ dli, T *__restrict__ dx,
                                                                     float *__restrict__ dh_pre, int64_t M, int n,
                                                                     int C) {
    const int lane = threadIdx.x & 63;
    for (int64_t t = (int64_t)blockIdx.x * kMixWaves + (threadIdx.x >> 6); t < M; t += (int64_t)gridDim.x * kMixWaves) {
        float hp[kMaxStreams], dh[kMaxStreams];
#pragma unroll
        for (int s = 0; s < kMaxStreams; ++s) {
            hp[s] = s < n ? h_pre[t * n + s] : 0.f;
            dh[s] = 0.f;
        }
        for (int c = 4 * lane; c < C; c += 256) {
            const f32x4 g = load4(dli + t * C + c);
#pragma unroll
            for (int s = 0; s < kMaxStreams; ++s) {
                if (s >= n) continue;
                const f32x4 xv = load4(x + (t * n + s) * C + c);
                dh[s] += g[0] * xv[0] + g[1] * xv[1] + g[2] * xv[2] + g[3] * xv[3];
                store4(dx + (t * n + s) * C + c, hp[s] * g);
            }
        }
#pragma unroll
        for (int s = 0; s < kMaxStreams; ++s) {
            if (s >= n) continue;
            const float v = wave_sum(dh[s]);
            if (lane == 0) dh_pre[t * n + s] = v;
        }
    }
}

template <typename T>
__global__ __launch_bounds__(64 * kMixWaves) void mhc_post_bwd_kernel(const T *__restrict__ x, const T *__restrict__ out,
                                                                      const float *__restrict__ h_res,
                                                                      const float *__restrict__ h_post,
                                                                      const T *__restrict__ dnew, T *__restrict__ dx,
                                                                      T *__restrict__ dout, float *__restrict__ dh_res,
                                                                      float *__restrict__ dh_post, int64_t M, int n,
                                                                      int C) {
    const int lane = threadIdx.x & 63;
    for (int64_t t = (int64_t)blockIdx.x * kMixWaves + (threadIdx.x >> 6); t < M; t += (int64_t)gridDim.x * kMixWaves) {
        float hr[kMaxStreams][kMaxStreams], hq[kMaxStreams];
        float dr[kMaxStreams][kMaxStreams], dq[kMaxStreams];
#pragma unroll
        for (int i = 0; i < kMaxStreams; ++i) {
            hq[i] = i < n ? h_post[t * n + i] : 0.f;
            dq[i] = 0.f;
#pragma unroll
            for (int s = 0; s < kMaxStreams; ++s) {
                hr[i][s] = (i < n && s < n) ? h_res[(t * n + i) * n + s] : 0.f;
                dr[i][s] = 0.f;
            }
        }
        for (int c = 4 * lane; c < C; c += 256) {
            f32x4 g[kMaxStreams], xv[kMaxStreams];
#pragma unroll
            for (int i = 0; i < kMaxStreams; ++i) {
                g[i] = i < n ? load4(dnew + (t * n + i) * C + c) : f32x4{0.f, 0.f, 0.f, 0.f};
                xv[i] = i < n ? load4(x + (t * n + i) * C + c) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
            const f32x4 o = load4(out + t * C + c);
            f32x4 go = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < kMaxStreams; ++i) {
                go += hq[i] * g[i];
                dq[i] += g[i][0] * o[0] + g[i][1] * o[1] + g[i][2] * o[2] + g[i][3] * o[3];
#pragma unroll
                for (int s = 0; s < kMaxStreams; ++s)
                    dr[i][s] += g[i][0] * xv[s][0] + g[i][1] * xv[s][1] + g[i][2] * xv[s][2] + g[i][3] * xv[s][3];
            }
            store4(dout + t * C + c, go);
#pragma unroll
            for (int s = 0; s < kMaxStreams; ++s) {
                if (s >= n) continue;
                f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < kMaxStreams; ++i) d += hr[i][s] * g[i];
                store4(dx + (t * n + s) * C + c, d);
            }
        }
#pragma unroll
        for (int i = 0; i < kMaxStreams; ++i) {
            if (i >= n) continue;
            const float vq = wave_sum(dq[i]);
            if (lane == 0) dh_post[t * n + i] = vq;
#pragma unroll
            for (int s = 0; s < kMaxStreams; ++s) {
                if (s >= n) continue;
                const float v = wave_sum(dr[i][s]);
                if (lane == 0) dh_res[(t * n + i) * n + s] = v;
            }
        }
    }
}

__global__ void sinkhorn_kernel(const float *__restrict__ h, int64_t batch, int n, int n_iter, float eps,
                                float *__restrict__ out) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < batch; b += (int64_t)gridDim.x * blockDim.x) {
        float m[8][8];
        const float *src = h + b * n * n;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) m[i][j] = (i < n && j < n) ? src[i * n + j] : 0.f;
        sinkhorn_regs<8>(m, n, n_iter, eps);
        float *dst = out + b * n * n;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (i < n && j < n) dst[i * n + j] = m[i][j];
    }
}

// ---------------------------------------------------------------- pre (mapping)
struct PreArgs {
    const void *x;
    int64_t ldx;
    int M, n, C;
    const void *phi;        // [32][n*C] activation dtype, rows: pre(n), post(n), res(n*n), zero pad
    const float *coef;      // alpha_pre, alpha_post, alpha_res
    const float *bias;      // pre[n], post[n], res[n*n]
    float rms_eps, sk_eps;
    int n_iter;
    float *h_pre, *h_post, *h_res;
    void *layer_in;
    int64_t ld_in;
};

// One workgroup = 32 tokens; wavefront w reduces the K range [w*K/4, (w+1)*K/4)
// (K = n*C) of the 32 x 32 projection D = x . phi^T on matrix cores, plus the
// per-token sum of squares.  The epilogue (one thread per token) applies the
// RMS scale, the sigmoid / 2*sigmoid / Sinkhorn constraints, and finally all
// threads form layer_in = sum_s H_pre[s] x[s, :] re-reading the (cache-hot) x.
template <typename T, bool BF16MMA>
__global__ __launch_bounds__(kPreThreads) void mhc_pre_kernel(PreArgs a) {
    __shared__ float part[kPreWaves][kPreTok][kPhiRows + 1];
    __shared__ float ssp[kPreWaves][kPreTok];
    __shared__ float hpre_s[kPreTok][kMaxStreams];

    constexpr uint32_t esz = sizeof(T);
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int m = lane & 15, kq = lane >> 4;
    const int n = a.n;
    const int K = n * a.C;
    const int tok0 = blockIdx.x * kPreTok;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * esz));
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.phi, (uint32_t)((int64_t)kPhiRows * K * esz));

    // wave's K slice, a multiple of 16
    const int kslice = (int)ceil_div(ceil_div(K, kPreWaves), 16) * 16;
    const int kbeg = wave * kslice;
    const int kend = min(K, kbeg + kslice);

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss[2] = {0.f, 0.f};
    uint32_t xrow[2];
    bool tok_ok[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int tok = tok0 + 16 * mt + m;
        tok_ok[mt] = tok < a.M;
        xrow[mt] = (uint32_t)((int64_t)tok * a.ldx * esz);
    }
    for (int k0 = kbeg; k0 < kend; k0 += 16) {
        const int k = k0 + 4 * kq;
        const bool kok = k < kend;  // K % 4 == 0, so a quad is all-in or all-out
        f32x4 xa[2], pb[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
            xa[mt] = Buf4<T>::load(xr, (kok && tok_ok[mt]) ? xrow[mt] + (uint32_t)k * esz : kOOB, 0);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
            pb[nt] = Buf4<T>::load(pr, kok ? (uint32_t)(((int64_t)(16 * nt + m) * K + k) * esz) : kOOB, 0);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            ss[mt] += xa[mt].x * xa[mt].x + xa[mt].y * xa[mt].y + xa[mt].z * xa[mt].z + xa[mt].w * xa[mt].w;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                if constexpr (BF16MMA) {
                    uint2 av, bv;
                    av.x = pack_bf16x2(xa[mt].x, xa[mt].y);
                    av.y = pack_bf16x2(xa[mt].z, xa[mt].w);
                    bv.x = pack_bf16x2(pb[nt].x, pb[nt].y);
                    bv.y = pack_bf16x2(pb[nt].z, pb[nt].w);
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        __builtin_bit_cast(i16x4, av), __builtin_bit_cast(i16x4, bv), acc[mt][nt], 0, 0, 0);
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        acc[mt][nt] =
                            __builtin_amdgcn_mfma_f32_16x16x4f32(xa[mt][s], pb[nt][s], acc[mt][nt], 0, 0, 0);
                }
            }
        }
    }
    // sum of squares: the 4 lanes (kq) of a token hold disjoint k quads
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        ss[mt] += __shfl_xor(ss[mt], 16);
        ss[mt] += __shfl_xor(ss[mt], 32);
    }
    if (kq == 0) {
        ssp[wave][m] = ss[0];
        ssp[wave][16 + m] = ss[1];
    }
    // D[token 4*kq + j][out m] of each (mt, nt) tile
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j) part[wave][16 * mt + 4 * kq + j][16 * nt + m] = acc[mt][nt][j];
    __syncthreads();

    if (tid < 4 * kPreTok) {
        const int t = tid >> 2, r = tid & 3;
        float ssum = 0.f;
#pragma unroll
        for (int w = 0; w < kPreWaves; ++w) ssum += ssp[w][t];
        const float rs = __fdiv_rn(1.0f, sqrtf(__fdiv_rn(ssum, (float)K) + a.rms_eps));
        auto dynf = [&](int o) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < kPreWaves; ++w) s += part[w][t][o];
            return s * rs;
        };
        token_constraints_quad(t, r, tok0 + t, a.M, n, a.coef, a.bias, a.n_iter, a.sk_eps, dynf, &hpre_s[0][0],
                               a.h_pre, a.h_post, a.h_res);
    }
    __syncthreads();

    // layer_in[t, c] = sum_s H_pre[t, s] x[t, s, c], 4 columns per item
    const int C = a.C;
    const int cq = C / 4;
    const __amdgpu_buffer_rsrc_t lr = make_rsrc(a.layer_in, (uint32_t)((int64_t)a.M * a.ld_in * esz));
    for (int item = tid; item < kPreTok * cq; item += kPreThreads) {
        const int t = item / cq;
        const int c = (item - t * cq) * 4;
        const int tok = tok0 + t;
        const bool ok = tok < a.M;
        const uint32_t xo = ok ? (uint32_t)(((int64_t)tok * a.ldx + c) * esz) : kOOB;
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < n; ++s) sum += hpre_s[t][s] * Buf4<T>::load(xr, xo, (uint32_t)(s * C) * esz);
        Buf4<T>::store(sum, lr, ok ? (uint32_t)(((int64_t)tok * a.ld_in + c) * esz) : kOOB, 0);
    }
}

// ---------------------------------------------------------------- pre, LDS-resident tile
// Same results as mhc_pre_kernel, for rows up to 8 KB: a workgroup keeps its
// whole tile of TT = 16*MT tokens (n*C values each) in LDS, so x is read
// from HBM once.  phi arrives in matrix-core fragment order
// ([K/16][2][64 lanes][4]: one coalesced 512-byte read per K step), the four
// wavefronts split K, partial projections meet in LDS, one thread per token
// runs the constraints, and layer_in (optionally RMS-normalised with a
// weight, the block's attention_norm / ffn_norm) is formed from LDS.
struct Pre2Args {
    const void *x;
    int64_t ldx;
    int M, n, C;
    const void *phi_frag;   // [K/16][2][64][4] activation dtype
    const float *coef, *bias;
    float rms_eps, sk_eps;
    int n_iter;
    float *h_pre, *h_post, *h_res;
    void *layer_in;
    int64_t ld_in;
    const float *norm_w;    // nullable: layer_in = rmsnorm(layer_in) * norm_w
    float norm_eps;
    // POST variant: the tile is the previous stream's update
    //   x_new[t, r, :] = sum_s hr_prev[t, r, s] xo[t, s, :] + hp_prev[t, r] out[t, :]
    // formed while it is loaded, kept in LDS and written to x_new (x unused)
    const void *xo;
    int64_t ld_xo;
    const void *out;
    int64_t ld_out;
    const float *hr_prev, *hp_prev;
    void *x_new;
    int64_t ld_new;
};

constexpr int kTileBytes = 128 * 1024;
constexpr int kPostItems = 4;             // POST: (token, 16-byte column chunk) items per thread per round

// FAST: n = 4 streams of C = 512 (n_embd 512), as compile-time constants.
template <typename T, bool BF16MMA, int MT, bool POST = false, bool FAST = false>
__global__ __launch_bounds__(kPreThreads, 2) void mhc_pre2_kernel(Pre2Args a) {
    constexpr int TT = 16 * MT;
    constexpr uint32_t esz = sizeof(T);
    extern __shared__ __align__(16) unsigned char smem[];
    const int n = FAST ? 4 : a.n, C = FAST ? 512 : a.C, K = n * C;
    const int rowb = K * (int)esz;
    const int stride = rowb + 8;              // 8-byte pad: 16 rows of a fragment read hit distinct banks
    unsigned char *xs = smem;                 // [TT][stride]
    float *part = (float *)(smem + TT * stride);              // [4][TT][33]
    float *ssp = part + kPreWaves * TT * (kPhiRows + 1);     // [4][TT]
    float *hpre = ssp + kPreWaves * TT;                      // [TT][4]
    f32x4 *nw_l = (f32x4 *)(hpre + TT * 4);                  // [C/4]

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tok0 = blockIdx.x * TT;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * esz));

    // phase 1 set-up (its first phi batch is requested before the tile lands)
    const int m = lane & 15, kq = lane >> 4;
    const int nks = K / 16;
    const int ks_per = (nks + kPreWaves - 1) / kPreWaves;
    const int ks0 = wave * ks_per, ks1 = min(nks, ks0 + ks_per);
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.phi_frag, (uint32_t)((int64_t)nks * 2 * 64 * 4 * esz));
    constexpr int kPf = 8;                    // K steps of phi per batch
    // phi fragments stay in the operand format: 4 bf16 (8 bytes) or 4 f32
    typedef typename std::conditional<BF16MMA, u32x2, f32x4>::type PhiT;
    PhiT pa[kPf][2], pbb[kPf][2];             // ping-pong buffers (static indexing keeps them in VGPRs)
    auto load_phi = [&](int kb, PhiT (&dst)[kPf][2]) {
#pragma unroll
        for (int u = 0; u < kPf; ++u)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int ks = kb + u;
                const uint32_t off = ks < ks1 ? (uint32_t)((((int64_t)ks * 2 + nt) * 64 + lane) * 4 * esz) : kOOB;
                if constexpr (BF16MMA)
                    dst[u][nt] = __builtin_amdgcn_raw_buffer_load_b64(pr, off, 0, 0);
                else
                    dst[u][nt] = Buf4<T>::load(pr, off, 0);
            }
    };
    // the norm weights (or ones), coef and bias go to LDS with the tile; they
    // are requested before the tile (C / 4 <= kPreThreads) and written once
    // it is in flight, so waiting for them does not wait for the tile
    // (buffer loads, zero past their ranges, with no branch around them and
    // no conversion until put_small: a branch or conversion right after a
    // load waits for every load issued before it)
    static_assert(1024 / 4 <= kPreThreads, "one norm-weight quad per thread");
    u32x4 nwr = {0u, 0u, 0u, 0u};
    if (a.norm_w)
        nwr = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(a.norm_w, (uint32_t)(C * 4)),
                                                    tid < C / 4 ? (uint32_t)(16 * tid) : kOOB, 0, 0);
    float *cb_l = (float *)(nw_l + C / 4);    // [3 coef][2n + n*n bias]
    const int ncb = 3 + 2 * n + n * n;
    const uint32_t cr = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(a.coef, 12u), tid < 3 ? (uint32_t)(4 * tid) : kOOB,
                                                             0, 0);
    const uint32_t br = __builtin_amdgcn_raw_buffer_load_b32(
        make_rsrc(a.bias, (uint32_t)((ncb - 3) * 4)), tid >= 3 && tid < ncb ? (uint32_t)(4 * (tid - 3)) : kOOB, 0, 0);
    auto put_small = [&]() {
        if (tid < C / 4) nw_l[tid] = a.norm_w ? __builtin_bit_cast(f32x4, nwr) : f32x4{1.f, 1.f, 1.f, 1.f};
        if (tid < ncb) cb_l[tid] = __uint_as_float(tid < 3 ? cr : br);
    };

    // phase 0 (POST): the stream update of the previous layer, formed per
    // (token, 16-byte column chunk) from the n old stream chunks and the
    // layer output chunk, in mhc_post_kernel's operation order (so x_new is
    // bitwise what that kernel writes); rounded to T, kept in LDS, stored.
    // The stores drain behind this phase's arithmetic (5 multiply-adds per
    // value) and the projection's first phi batch, which was requested
    // before them.
    if constexpr (POST) {
        const int cpc = C * (int)esz / 16;    // chunks per stream row
        const int nit = TT * cpc;
        const int nh = n * n + n;
        float *hprev = part;                  // [TT][n*n + n]; part is free until phase 1 ends
        const __amdgpu_buffer_rsrc_t xor_ = make_rsrc(a.xo, (uint32_t)((int64_t)a.M * a.ld_xo * esz));
        const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out, (uint32_t)((int64_t)a.M * a.ld_out * esz));
        const __amdgpu_buffer_rsrc_t nr = make_rsrc(a.x_new, (uint32_t)((int64_t)a.M * a.ld_new * esz));
        u32x4 xv[kPostItems][kMaxStreams], ov[kPostItems];
        auto load_round = [&](int it0) {
#pragma unroll
            for (int i = 0; i < kPostItems; ++i) {
                const int it = it0 + tid + i * kPreThreads;
                const int r = it / cpc, cc = it - r * cpc;
                const bool ok = it < nit && tok0 + r < a.M;
#pragma unroll
                for (int st = 0; st < kMaxStreams; ++st)
                    xv[i][st] = __builtin_amdgcn_raw_buffer_load_b128(
                        xor_, ok && st < n ? (uint32_t)(((int64_t)(tok0 + r) * a.ld_xo + st * C) * esz + cc * 16) : kOOB,
                        0, 0);
                ov[i] = __builtin_amdgcn_raw_buffer_load_b128(
                    orr, ok ? (uint32_t)((int64_t)(tok0 + r) * a.ld_out * esz + cc * 16) : kOOB, 0, 0);
            }
        };
        // the previous H_res / H_post rows of the tile are requested first, so
        // the barrier waits for them alone and each item below waits only for
        // its own loads
        constexpr int kMaxH = (TT * (kMaxStreams * kMaxStreams + kMaxStreams) + kPreThreads - 1) / kPreThreads;
        uint32_t hvr[kMaxH], hvp[kMaxH];
        {
            const __amdgpu_buffer_rsrc_t hrr = make_rsrc(a.hr_prev, (uint32_t)((int64_t)a.M * n * n * 4));
            const __amdgpu_buffer_rsrc_t hpr = make_rsrc(a.hp_prev, (uint32_t)((int64_t)a.M * n * 4));
#pragma unroll
            for (int i = 0; i < kMaxH; ++i) {
                const int e = tid + i * kPreThreads;
                const int r = e / nh, k = e - r * nh;
                const bool ok = e < TT * nh && tok0 + r < a.M;
                hvr[i] = __builtin_amdgcn_raw_buffer_load_b32(
                    hrr, ok && k < n * n ? (uint32_t)(((int64_t)(tok0 + r) * n * n + k) * 4) : kOOB, 0, 0);
                hvp[i] = __builtin_amdgcn_raw_buffer_load_b32(
                    hpr, ok && k >= n * n ? (uint32_t)(((int64_t)(tok0 + r) * n + (k - n * n)) * 4) : kOOB, 0, 0);
            }
        }
        load_round(0);
        load_phi(ks0, pa);
        put_small();
#pragma unroll
        for (int i = 0; i < kMaxH; ++i) {
            const int e = tid + i * kPreThreads;
            const int k = e - (e / nh) * nh;
            if (e < TT * nh) hprev[e] = __uint_as_float(k < n * n ? hvr[i] : hvp[i]);
        }
        lds_barrier();
        constexpr int VE = 16 / (int)esz;     // values per chunk: 8 bf16 or 4 f32
        for (int it0 = 0; it0 < nit; it0 += kPostItems * kPreThreads) {
            if (it0) load_round(it0);
#pragma unroll
            for (int i = 0; i < kPostItems; ++i) {
                const int it = it0 + tid + i * kPreThreads;
                if (it >= nit) continue;
                const int r = it / cpc, cc = it - r * cpc;
                const bool ok = tok0 + r < a.M;
                const float *hr = hprev + r * nh, *hp = hr + n * n;
                float xf[kMaxStreams][8], of[8];
                auto unpack = [&](const u32x4 &u, float (&f)[8]) {
                    if constexpr (sizeof(T) == 2) {
                        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            f[2 * q] = __uint_as_float(w[q] << 16);
                            f[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
                        }
                    } else {
                        f[0] = __uint_as_float(u.x);
                        f[1] = __uint_as_float(u.y);
                        f[2] = __uint_as_float(u.z);
                        f[3] = __uint_as_float(u.w);
                    }
                };
#pragma unroll
                for (int st = 0; st < kMaxStreams; ++st) unpack(xv[i][st], xf[st]);
                unpack(ov[i], of);
#pragma unroll
                for (int rr = 0; rr < kMaxStreams; ++rr) {
                    if (rr >= n) continue;
                    float acc[8];
#pragma unroll
                    for (int e = 0; e < VE; ++e) acc[e] = hp[rr] * of[e];
#pragma unroll
                    for (int st = 0; st < kMaxStreams; ++st) {
                        if (st >= n) continue;
                        const float h = hr[rr * n + st];
#pragma unroll
                        for (int e = 0; e < VE; ++e) acc[e] += h * xf[st][e];
                    }
                    u32x4 pk;
                    if constexpr (sizeof(T) == 2) {
                        pk = u32x4{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                                   pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7])};
                    } else {
                        pk = u32x4{__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]),
                                   __float_as_uint(acc[3])};
                    }
                    u32x2 *d = (u32x2 *)(xs + r * stride + rr * C * esz + cc * 16);
                    d[0] = u32x2{pk.x, pk.y};
                    d[1] = u32x2{pk.z, pk.w};
                    __builtin_amdgcn_raw_buffer_store_b128(
                        pk, nr, ok ? (uint32_t)(((int64_t)(tok0 + r) * a.ld_new + rr * C) * esz + cc * 16) : kOOB,
                        0, 0);
                }
            }
        }
    } else
    // phase 0: tile -> LDS, all 16-byte loads in flight together
    {
        const int cpr = rowb / 16;            // chunks per row
        const int nch = TT * cpr;
        const bool pow2 = (cpr & (cpr - 1)) == 0;
        const int lg = 31 - __builtin_clz(cpr);
        constexpr int kMaxPer = kTileBytes / 16 / kPreThreads;   // 32
        u32x4 st[kMaxPer];
#pragma unroll
        for (int j = 0; j < kMaxPer; ++j) {
            const int ch = tid + j * kPreThreads;
            const int r = pow2 ? (ch >> lg) : ch / cpr, cc = ch - r * cpr;
            const bool ok = ch < nch && tok0 + r < a.M;
            st[j] = __builtin_amdgcn_raw_buffer_load_b128(
                xr, ok ? (uint32_t)(((int64_t)(tok0 + r) * a.ldx) * esz + cc * 16) : kOOB, 0, 0);
        }
        load_phi(ks0, pa);
        put_small();
#pragma unroll
        for (int j = 0; j < kMaxPer; ++j) {
            const int ch = tid + j * kPreThreads;
            if (ch < nch) {
                const int r = pow2 ? (ch >> lg) : ch / cpr, cc = ch - r * cpr;
                u32x2 *d = (u32x2 *)(xs + r * stride + cc * 16);
                d[0] = u32x2{st[j].x, st[j].y};
                d[1] = u32x2{st[j].z, st[j].w};
            }
        }
    }
    // LDS only: the x_new stores (POST) and the first phi batch stay in flight
    lds_barrier();

    // phase 1: projection on matrix cores, K split over the 4 wavefronts
    f32x4 acc[MT][2], accss[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i][0] = acc[i][1] = accss[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) ss[i] = 0.f;
    auto compute = [&](int kb, const PhiT (&p)[kPf][2]) {
#pragma unroll
        for (int u = 0; u < kPf; ++u) {
            const int ks = kb + u;
            if (ks >= ks1) break;
            const int k = ks * 16 + 4 * kq;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const unsigned char *src = xs + (16 * mt + m) * stride + k * esz;
                if constexpr (BF16MMA) {
                    // raw bf16 operands; the sum of squares is the diagonal of x x^T
                    const i16x4 xr4 = __builtin_bit_cast(i16x4, *(const u32x2 *)src);
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                            xr4, __builtin_bit_cast(i16x4, p[u][nt]), acc[mt][nt], 0, 0, 0);
                    accss[mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(xr4, xr4, accss[mt], 0, 0, 0);
                    continue;
                }
                f32x4 xa;
                if constexpr (sizeof(T) == 2) {
                    const u32x2 u2 = *(const u32x2 *)src;
                    xa.x = __uint_as_float(u2.x << 16);
                    xa.y = __uint_as_float(u2.x & 0xffff0000u);
                    xa.z = __uint_as_float(u2.y << 16);
                    xa.w = __uint_as_float(u2.y & 0xffff0000u);
                } else {
                    const u32x2 lo = *(const u32x2 *)src, hi = *(const u32x2 *)(src + 8);
                    xa = __builtin_bit_cast(f32x4, u32x4{lo.x, lo.y, hi.x, hi.y});
                }
                ss[mt] += xa.x * xa.x + xa.y * xa.y + xa.z * xa.z + xa.w * xa.w;
                if constexpr (!BF16MMA) {
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                        for (int s2 = 0; s2 < 4; ++s2)
                            acc[mt][nt] =
                                __builtin_amdgcn_mfma_f32_16x16x4f32(xa[s2], p[u][nt][s2], acc[mt][nt], 0, 0, 0);
                }
            }
        }
    };
    for (int kb = ks0; kb < ks1; kb += 2 * kPf) {
        if (kb + kPf < ks1) load_phi(kb + kPf, pbb);
        compute(kb, pa);
        if (kb + kPf < ks1) {
            if (kb + 2 * kPf < ks1) load_phi(kb + 2 * kPf, pa);
            compute(kb + kPf, pbb);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if constexpr (BF16MMA) {
            // lane (n = m, q = kq) holds rows 4kq..4kq+3 of column m of x x^T
            const int j = m - 4 * kq;
            if (j >= 0 && j < 4) ssp[wave * TT + 16 * mt + m] = accss[mt][j];
        } else {
            ss[mt] += __shfl_xor(ss[mt], 16);
            ss[mt] += __shfl_xor(ss[mt], 32);
            if (kq == 0) ssp[wave * TT + 16 * mt + m] = ss[mt];
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                part[(wave * TT + 16 * mt + 4 * kq + j) * (kPhiRows + 1) + 16 * nt + m] = acc[mt][nt][j];
    }
    lds_barrier();

    // phases 2 and 3, one group of 4 tokens per wavefront: lane l serves
    // token t = 4 wave + l / 16.
    //   constraints: each quad of the token's 16 lanes runs them (lane row
    //     r = l % 4); the four quads compute the same values, the first stores.
    //   layer_in = sum_s H_pre[s] x[s, :]: 16 lanes per token, 4 values per
    //     item (H_pre from the lane's quad), optionally RMS-normalised over
    //     the row with weight norm_w.
    // The Sinkhorn iterations, a dependent chain of quad shuffles and
    // reciprocals, are interleaved with the layer_in items, one item per
    // iteration, so that the items' arithmetic fills the chain's latency.
    static_assert(MT == 1, "one 16-token tile: 4 wavefronts x 4 tokens");
    {
        const int gt = 4 * wave + (lane >> 4), gr = lane & 3, sub = lane & 15;
        float ssum = 0.f;
#pragma unroll
        for (int w = 0; w < kPreWaves; ++w) ssum += ssp[w * TT + gt];
        const float rs = __fdiv_rn(1.0f, sqrtf(__fdiv_rn(ssum, (float)K) + a.rms_eps));
        auto dynf = [&](int o) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < kPreWaves; ++w) s += part[(w * TT + gt) * (kPhiRows + 1) + o];
            return s * rs;
        };
        QuadGates gq = token_gates_quad(gr, n, cb_l, cb_l + 3, dynf);
        const float hp[kMaxStreams] = {quad_bcast<0>(gq.pre), quad_bcast<1>(gq.pre), quad_bcast<2>(gq.pre),
                                       quad_bcast<3>(gq.pre)};
        constexpr int KQ = FAST ? 8 : 1024 / 4 / 16;   // items per lane (C <= 1024)
        const int nq = C / 4;
        f32x4 v[KQ];
        float sq = 0.f;
#pragma unroll
        for (int j = 0; j < KQ; ++j) {
            {
                float mn[kMaxStreams];
#pragma unroll
                for (int i = 0; i < kMaxStreams; ++i) mn[i] = gq.m[i];
                sinkhorn_quad_step(mn, n, a.sk_eps);
                const bool live = j < a.n_iter;
#pragma unroll
                for (int i = 0; i < kMaxStreams; ++i) gq.m[i] = live ? mn[i] : gq.m[i];
            }
            const int q = sub + 16 * j;
            const bool qok = q < nq;
            const int qc = qok ? q : 0;
            f32x4 acc4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < kMaxStreams; ++s) {
                if (s >= n) continue;
                const unsigned char *src = xs + gt * stride + (s * C + 4 * qc) * esz;
                f32x4 xv;
                if constexpr (sizeof(T) == 2) {
                    const u32x2 u2 = *(const u32x2 *)src;
                    xv.x = __uint_as_float(u2.x << 16);
                    xv.y = __uint_as_float(u2.x & 0xffff0000u);
                    xv.z = __uint_as_float(u2.y << 16);
                    xv.w = __uint_as_float(u2.y & 0xffff0000u);
                } else {
                    const u32x2 lo = *(const u32x2 *)src, hi = *(const u32x2 *)(src + 8);
                    xv = __builtin_bit_cast(f32x4, u32x4{lo.x, lo.y, hi.x, hi.y});
                }
                acc4 += hp[s] * xv;
            }
            if (!qok) acc4 = f32x4{0.f, 0.f, 0.f, 0.f};
            v[j] = acc4;
            sq += acc4.x * acc4.x + acc4.y * acc4.y + acc4.z * acc4.z + acc4.w * acc4.w;
        }
        for (int it = KQ; it < a.n_iter; ++it) sinkhorn_quad_step(gq.m, n, a.sk_eps);
        if (((lane >> 2) & 3) == 0)
            token_store_quad(gq, gr, tok0 + gt, a.M, n, a.h_pre, a.h_post, a.h_res);

        float scale = 1.f;
        if (a.norm_w) {
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) sq += __shfl_xor(sq, sh);
            scale = 1.0f / sqrtf(__fdiv_rn(sq, (float)C) + a.norm_eps);
        }
        const __amdgpu_buffer_rsrc_t lr = make_rsrc(a.layer_in, (uint32_t)((int64_t)a.M * a.ld_in * esz));
        const int tok = tok0 + gt;
        const bool ok = tok < a.M;
#pragma unroll
        for (int j = 0; j < KQ; ++j) {
            const int q = sub + 16 * j;
            const f32x4 o = v[j] * scale * nw_l[q < nq ? q : 0];
            Buf4<T>::store(o, lr, ok && q < nq ? (uint32_t)(((int64_t)tok * a.ld_in + 4 * q) * esz) : kOOB, 0);
        }
    }
}

// ---------------------------------------------------------------- pre, wide rows
// ResidualStreamMapping x3 + H_pre @ x (+ the block's RMSNorm) for rows too
// long for an LDS tile (n*C up to 16384: n_embd 4096), in two launches:
//   mhc_proj_kernel   one wavefront per (16-token tile, K split): streams the
//                     rows through 16x16x32 matrix-core steps against the
//                     projection (phi fragments [K/32][2][64][8]) and the
//                     x x^T diagonal (sum of squares); writes partial sums
//                     [split][M][25] (24 projections + sum of squares);
//   mhc_apply_kernel  one wavefront per token: sums the splits, RMS scale,
//                     the constraints (4-lane Sinkhorn), then layer_in =
//                     sum_s H_pre[s] x[s, :] with its RMS norm over C.
// Small batches (decode) split K across many wavefronts; prefill uses one
// split, so each row is read twice (projection, apply).
constexpr int kProjOut = kPhiRows - 8 + 1;  // 24 projection outputs + sum of squares

struct ProjArgs {
    const void *x;
    int64_t ldx;
    int M, K, splits, kper;   // kper: K per split (multiple of 32)
    const void *phi32;        // [K/32][2][64][8] activation dtype
    float *part;              // [splits][M][25]
};

template <typename T>
__global__ __launch_bounds__(256) void mhc_proj_kernel(ProjArgs a) {
    constexpr uint32_t esz = sizeof(T);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4;
    const int n_tiles = (int)ceil_div(a.M, 16);
    const int item = blockIdx.x * 4 + wave;
    if (item >= n_tiles * a.splits) return;
    const int tile = item / a.splits, split = item % a.splits;
    const int k0 = split * a.kper, k1 = min(a.K, k0 + a.kper);
    const int tok = tile * 16 + m;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * esz));
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.phi32, (uint32_t)((int64_t)a.K * 32 * esz));
    const uint32_t xrow = tok < a.M ? (uint32_t)((int64_t)tok * a.ldx * esz) : kOOB;
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}, accss = {0.f, 0.f, 0.f, 0.f};
    if constexpr (sizeof(T) == 2) {
        // batches of kU steps: all loads of a batch are issued before its products
        constexpr int kU = 8;
        for (int kb = k0; kb < k1; kb += 32 * kU) {
            u32x4 xv[kU], pv[kU][2];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int k = kb + 32 * u;
                const bool ok = k < k1;
                const uint32_t xo = (xrow == kOOB || !ok) ? kOOB : xrow + (uint32_t)(k + 8 * kq) * esz;
                xv[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 0, 0);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const uint32_t po =
                        ok ? (uint32_t)((((int64_t)(k / 32) * 2 + nt) * 64 + lane) * 8 * esz) : kOOB;
                    pv[u][nt] = __builtin_amdgcn_raw_buffer_load_b128(pr, po, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const bf16x8 x8 = __builtin_bit_cast(bf16x8, xv[u]);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, __builtin_bit_cast(bf16x8, pv[u][nt]),
                                                                      acc[nt], 0, 0, 0);
                accss = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, x8, accss, 0, 0, 0);
            }
        }
    } else
    for (int k = k0; k < k1; k += 32) {
        const uint32_t xo = xrow == kOOB ? kOOB : xrow + (uint32_t)(k + 8 * kq) * esz;
        const uint32_t po = (uint32_t)(((int64_t)(k / 32) * 2 * 64 + lane) * 8 * esz);
        {
            const f32x4 x0 = Buf4<float>::load(xr, xo, 0), x1 = Buf4<float>::load(xr, xo, 16);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t pn = po + (uint32_t)nt * 64 * 8 * esz;
                const f32x4 p0 = Buf4<float>::load(pr, pn, 0), p1 = Buf4<float>::load(pr, pn, 16);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0[u], p0[u], acc[nt], 0, 0, 0);
                    acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1[u], p1[u], acc[nt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                accss = __builtin_amdgcn_mfma_f32_16x16x4f32(x0[u], x0[u], accss, 0, 0, 0);
                accss = __builtin_amdgcn_mfma_f32_16x16x4f32(x1[u], x1[u], accss, 0, 0, 0);
            }
        }
    }
    // lane (n = m, q = kq) holds rows 4kq..4kq+3 (tokens) of column m (output)
    float *dst = a.part + (int64_t)split * a.M * kProjOut;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int o = 16 * nt + m;
        if (o >= kProjOut - 1) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = tile * 16 + 4 * kq + j;
            if (t < a.M) dst[(int64_t)t * kProjOut + o] = acc[nt][j];
        }
    }
    const int j = m - 4 * kq;
    if (j >= 0 && j < 4 && tile * 16 + m < a.M) dst[(int64_t)(tile * 16 + m) * kProjOut + kProjOut - 1] = accss[j];
}

// The previous stream's update fused into the projection (bf16): the same
// work items, but a K split is a range of columns c of every stream, and the
// lane's 8 columns of stream r are formed as mhc_post_kernel forms them
// (x_new[t, r, c] = H_post[t, r] out[t, c] + sum_s H_res[t, r, s] x[t, s, c],
// in that operation order, rounded to bf16), stored once, and fed to the
// products from registers.  The rows are read once, not three times (update
// read, update write, projection read); the products run c-major over the
// streams, so the partial sums are those of mhc_proj_kernel on x_new up to
// the order of the float32 accumulation.
struct PostProjArgs {
    const uint16_t *xo;       // previous streams [M, ld_xo]
    int64_t ld_xo;
    const uint16_t *out;      // the layer's output [M, ld_out]
    int64_t ld_out;
    const float *hr_prev, *hp_prev;  // [M, n, n], [M, n]
    uint16_t *x_new;          // [M, ld_new]
    int64_t ld_new;
    int M, n, C, splits, cper;  // cper: columns per split (multiple of 32)
    const uint16_t *phi32;    // [K/32][2][64][8]
    float *part;              // [splits][M][25]
};

// Every argument read at entry in one batch of scalar loads, the values kept
// through an empty asm statement: left to itself the compiler reads each
// field where it is first used, one memory round trip after another.
__device__ __forceinline__ PostProjArgs load_args(const PostProjArgs &src) {
    PostProjArgs a = src;
    asm volatile("" : "+s"(a.xo), "+s"(a.ld_xo), "+s"(a.out), "+s"(a.ld_out), "+s"(a.hr_prev), "+s"(a.hp_prev),
                 "+s"(a.x_new), "+s"(a.ld_new), "+s"(a.M), "+s"(a.n), "+s"(a.C), "+s"(a.splits), "+s"(a.cper),
                 "+s"(a.phi32), "+s"(a.part));
    return a;
}

// One 32-column block of a work item's loads: the lane's 8 columns of each
// previous stream and of the layer output, and the phi fragments of those
// columns for each new stream.
template <int N>
struct PostProjBlock {
    u32x4 x[N], o, p[N][2];
};

// No bounds selects: rows past M lie past the end of the x / out buffers
// (which end at row M) and load zeros; a block at or past the split's end
// (a prefetch beyond the last block) loads whatever lies there, within or
// past the buffers, and is never formed.
template <int N>
__device__ __forceinline__ void post_proj_load(PostProjBlock<N> &b, const PostProjArgs &a,
                                               __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t orr,
                                               __amdgpu_buffer_rsrc_t pr, uint32_t xrow, uint32_t orow, int c, int kq,
                                               int lane) {
    const uint32_t co = (uint32_t)(c + 8 * kq) * 2;
#pragma unroll
    for (int s2 = 0; s2 < N; ++s2)
        b.x[s2] = __builtin_amdgcn_raw_buffer_load_b128(xr, xrow + (uint32_t)(s2 * a.C) * 2 + co, 0, 0);
    b.o = __builtin_amdgcn_raw_buffer_load_b128(orr, orow + co, 0, 0);
#pragma unroll
    for (int r = 0; r < N; ++r)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
            b.p[r][nt] = __builtin_amdgcn_raw_buffer_load_b128(
                pr, (uint32_t)(((((r * a.C + c) >> 5) * 2 + nt) * 64 + lane) * 16), 0, 0);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Forms block d (0 or 1) of a pair of 32-column blocks: x_new goes to the
// wave's LDS stage (row m at m * kStagePitch, block d at byte 64 d) and to
// the matrix cores.
constexpr int kStagePitch = 2 * 64 + 16;   // two blocks of a row + 16 bytes (conflict-free writes)

template <int N>
__device__ __forceinline__ void post_proj_block(const PostProjBlock<N> &b, const float (&hr)[N][N],
                                                const float (&hp)[N], uint8_t *stage, int d, int m, int kq,
                                                f32x4 (&acc)[2], f32x4 &accss) {
#pragma unroll
    for (int r = 0; r < N; ++r) {
        uint32_t w[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            // columns 2d, 2d + 1 of the lane's 8, in mhc_post_kernel's operation order
            const uint32_t ow = d == 0 ? b.o.x : d == 1 ? b.o.y : d == 2 ? b.o.z : b.o.w;
            float lo = hp[r] * bf16_lo(ow), hi = hp[r] * bf16_hi(ow);
#pragma unroll
            for (int s2 = 0; s2 < N; ++s2) {
                const uint32_t xw = d == 0 ? b.x[s2].x : d == 1 ? b.x[s2].y : d == 2 ? b.x[s2].z : b.x[s2].w;
                lo += hr[r][s2] * bf16_lo(xw);
                hi += hr[r][s2] * bf16_hi(xw);
            }
            w[d] = pack_bf16x2(lo, hi);
        }
        const u32x4 nb = {w[0], w[1], w[2], w[3]};
        *(u32x4 *)(stage + (r * 16 + m) * kStagePitch + 64 * d + 16 * kq) = nb;
        // rows past M hold zeros (the loads gave zeros)
        const bf16x8 x8 = __builtin_bit_cast(bf16x8, nb);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
            acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, __builtin_bit_cast(bf16x8, b.p[r][nt]), acc[nt], 0,
                                                              0, 0);
        accss = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, x8, accss, 0, 0, 0);
    }
}

// Stores a pair of blocks from the wave's LDS stage: each store instruction
// covers 8 rows x 128 contiguous bytes (whole cache lines; stores of 64-byte
// halves a block apart write HBM at a fraction of its rate).
template <int N>
__device__ __forceinline__ void post_proj_flush(const uint8_t *stage, const PostProjArgs &a,
                                                __amdgpu_buffer_rsrc_t nr, int tile, int cb, int c1, int lane) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int chunk = lane & 7;             // 16-byte chunk of the row's 128 bytes
    const bool cok = cb + 32 * (chunk >> 2) < c1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = 8 * i + (lane >> 3), t = tile * 16 + row;
        const uint32_t nrow = t < a.M ? (uint32_t)((int64_t)t * a.ld_new * 2) : kOOB;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            const u32x4 v = *(const u32x4 *)(stage + (r * 16 + row) * kStagePitch + 16 * chunk);
            __builtin_amdgcn_raw_buffer_store_b128(
                v, nr, (nrow == kOOB || !cok) ? kOOB : nrow + (uint32_t)(r * a.C + cb + 8 * chunk) * 2, 0, 0);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int N>
__global__ __launch_bounds__(256) void mhc_post_proj_kernel(PostProjArgs args) {
    const PostProjArgs a = load_args(args);
    __shared__ __attribute__((aligned(16))) uint8_t stage_all[4][N * 16 * kStagePitch];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, m = lane & 15,
              kq = lane >> 4;
    const int n_tiles = (int)ceil_div(a.M, 16);
    const int item = blockIdx.x * 4 + wave;
    if (item >= n_tiles * a.splits) return;
    const int tile = item / a.splits, split = item % a.splits;
    const int C = a.C, K = N * C;
    const int c0 = split * a.cper, c1 = min(C, c0 + a.cper);
    const int tok = tile * 16 + m;
    const bool ok = tok < a.M;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xo, (uint32_t)((int64_t)a.M * a.ld_xo * 2));
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out, (uint32_t)((int64_t)a.M * a.ld_out * 2));
    const __amdgpu_buffer_rsrc_t nr = make_rsrc(a.x_new, (uint32_t)((int64_t)a.M * a.ld_new * 2));
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.phi32, (uint32_t)((int64_t)K * 32 * 2));
    // (tok < M + 16 and both buffers below 2^31 bytes: these offsets do not wrap)
    const uint32_t xrow = (uint32_t)((int64_t)tok * a.ld_xo * 2);
    const uint32_t orow = (uint32_t)((int64_t)tok * a.ld_out * 2);
    uint8_t *stage = stage_all[wave];
    // this lane's token's update coefficients, then the first two blocks'
    // loads (issued after the coefficients', so that the wait at the head
    // of the loop counts only block loads)
    // (buffer loads, zero past M: no branch around them, so none waits)
    float hr[N][N], hp[N];
    {
        const __amdgpu_buffer_rsrc_t hrr = make_rsrc(a.hr_prev, (uint32_t)((int64_t)a.M * N * N * 4));
        const __amdgpu_buffer_rsrc_t hpr = make_rsrc(a.hp_prev, (uint32_t)((int64_t)a.M * N * 4));
        const uint32_t ho = ok ? (uint32_t)tok * (N * N * 4) : kOOB, po = ok ? (uint32_t)tok * (N * 4) : kOOB;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            hp[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(hpr, po, r * 4, 0));
#pragma unroll
            for (int s2 = 0; s2 < N; ++s2)
                hr[r][s2] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(hrr, ho, (r * N + s2) * 4, 0));
        }
    }
    PostProjBlock<N> b0, b1;
    __builtin_amdgcn_sched_barrier(0);
    post_proj_load<N>(b0, a, xr, orr, pr, xrow, orow, c0, kq, lane);
    __builtin_amdgcn_sched_barrier(0);
    post_proj_load<N>(b1, a, xr, orr, pr, xrow, orow, c0 + 32, kq, lane);
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}, accss = {0.f, 0.f, 0.f, 0.f};
    // two blocks in flight: a block's loads are issued while the block
    // before it is formed, stored and multiplied.  No branches around them
    // (a block past c1 loads zeros, stores nothing and adds zeros), so the
    // compiler's wait before each block counts only that block's loads.
    // (scheduling barriers keep the compiler from merging the two blocks'
    // work and issuing both blocks' loads after it)
    for (int cb = c0; cb < c1; cb += 64) {
        post_proj_block<N>(b0, hr, hp, stage, 0, m, kq, acc, accss);
        __builtin_amdgcn_sched_barrier(0);
        post_proj_load<N>(b0, a, xr, orr, pr, xrow, orow, cb + 64, kq, lane);
        __builtin_amdgcn_sched_barrier(0);
        if (cb + 32 < c1) post_proj_block<N>(b1, hr, hp, stage, 1, m, kq, acc, accss);
        __builtin_amdgcn_sched_barrier(0);
        post_proj_load<N>(b1, a, xr, orr, pr, xrow, orow, cb + 96, kq, lane);
        __builtin_amdgcn_sched_barrier(0);
        post_proj_flush<N>(stage, a, nr, tile, cb, c1, lane);
        __builtin_amdgcn_sched_barrier(0);
    }
    // lane (n = m, q = kq) holds rows 4kq..4kq+3 (tokens) of column m (output)
    float *dst = a.part + (int64_t)split * a.M * kProjOut;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int o = 16 * nt + m;
        if (o >= kProjOut - 1) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = tile * 16 + 4 * kq + j;
            if (t < a.M) dst[(int64_t)t * kProjOut + o] = acc[nt][j];
        }
    }
    const int j = m - 4 * kq;
    if (j >= 0 && j < 4 && tile * 16 + m < a.M) dst[(int64_t)(tile * 16 + m) * kProjOut + kProjOut - 1] = accss[j];
}

struct ApplyArgs {
    const void *x;
    int64_t ldx;
    int M, n, C, splits;
    const float *part;        // [splits][M][25]
    const float *coef, *bias;
    float rms_eps, sk_eps;
    int n_iter;
    float *h_pre, *h_post, *h_res;
    void *layer_in;
    int64_t ld_in;
    const float *norm_w;
    float norm_eps;
};

template <typename T>
__global__ __launch_bounds__(256) void mhc_apply_kernel(ApplyArgs a) {
    constexpr uint32_t esz = sizeof(T);
    constexpr int kMaxQ = 16;                 // C <= 4096: 16 quads per lane
    __shared__ float dyn_s[4][kProjOut + 7];
    __shared__ float hpre_s[4][4];
    __shared__ float par_s[4][32];            // coef[3], then bias[2n + n*n]
    __shared__ float red_s[4][64][kProjOut];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tok = blockIdx.x * 4 + wave;
    const bool live = tok < a.M;
    const int n = a.n, C = a.C, K = n * C;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * esz));
    const int nq = C / 4;
    // the K split partials (splits <= 64: lane l holds split l) and the
    // mapping parameters are requested before the row: loads complete in
    // order, so waiting for them then does not wait for the row
    float pv[kProjOut];
    {
        const bool has = live && lane < a.splits;
        const float *src = a.part + ((int64_t)(has ? lane : 0) * a.M + (live ? tok : 0)) * kProjOut;
#pragma unroll
        for (int o = 0; o < kProjOut; ++o) pv[o] = has ? src[o] : 0.f;
    }
    const int n_par = 3 + 2 * n + n * n;
    const float par = lane < 3 ? a.coef[lane] : lane < n_par ? a.bias[lane - 3] : 0.f;
    // bf16: the token's whole row (n x C <= 16384 values, 128 registers per
    // lane) is requested next, 16 bytes (8 columns) per lane and load, so its
    // round trip overlaps the split sums and the constraints below
    constexpr int kRawO = sizeof(T) == 2 ? kMaxQ / 2 : 1;
    u32x4 raw[kRawO][kMaxStreams];
    if constexpr (sizeof(T) == 2) {
        const uint32_t xrow0 = live ? (uint32_t)((int64_t)tok * a.ldx * esz) : kOOB;
#pragma unroll
        for (int j = 0; j < kRawO; ++j) {
            const int c8 = 8 * (lane + 64 * j);
#pragma unroll
            for (int s = 0; s < kMaxStreams; ++s)
                raw[j][s] = __builtin_amdgcn_raw_buffer_load_b128(
                    xr, (xrow0 == kOOB || s >= n || c8 >= C) ? kOOB : xrow0 + (uint32_t)(s * C + c8) * esz, 0, 0);
        }
    }
    // sum the splits: lane o < 25 adds the 64 lane values from LDS in lane
    // (split) order
#pragma unroll
    for (int o = 0; o < kProjOut; ++o) red_s[wave][lane][o] = pv[o];
    if (lane < n_par) par_s[wave][lane] = par;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < kProjOut) {
        const int nl = a.splits < 64 ? a.splits : 64;
        float sum = 0.f;
        for (int l = 0; l < nl; ++l) sum += red_s[wave][l][lane];
        dyn_s[wave][lane] = sum;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 4) {
        const float rs = __fdiv_rn(1.0f, sqrtf(__fdiv_rn(dyn_s[wave][kProjOut - 1], (float)K) + a.rms_eps));
        auto dynf = [&](int o) { return dyn_s[wave][o] * rs; };
        token_constraints_quad(wave, lane, live ? tok : a.M, a.M, n, &par_s[wave][0], &par_s[wave][3], a.n_iter,
                               a.sk_eps, dynf, &hpre_s[0][0], a.h_pre, a.h_post, a.h_res);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (!live) return;
    float hp[kMaxStreams];
#pragma unroll
    for (int s = 0; s < kMaxStreams; ++s) hp[s] = hpre_s[wave][s];
    const __amdgpu_buffer_rsrc_t lr = make_rsrc(a.layer_in, (uint32_t)((int64_t)a.M * a.ld_in * esz));
    const uint32_t xrow = (uint32_t)((int64_t)tok * a.ldx * esz);
    // quad j of the lane: columns 4 q .. 4 q + 3 (bf16: the halves of the
    // lane's 8-column groups, q = 2 (lane + 64 (j / 2)) + j % 2)
    auto quad = [&](int j) { return sizeof(T) == 2 ? 2 * (lane + 64 * (j >> 1)) + (j & 1) : lane + 64 * j; };
    f32x4 v[kMaxQ];
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxQ; ++j) {
        const int q = quad(j);
        f32x4 acc4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kMaxStreams; ++s) {
            if (s >= n) continue;
            f32x4 xv;
            if constexpr (sizeof(T) == 2) {
                const u32x4 u = raw[j >> 1][s];
                const uint32_t u0 = (j & 1) ? u.z : u.x, u1 = (j & 1) ? u.w : u.y;
                xv = f32x4{__uint_as_float(u0 << 16), __uint_as_float(u0 & 0xffff0000u),
                           __uint_as_float(u1 << 16), __uint_as_float(u1 & 0xffff0000u)};
            } else {
                xv = Buf4<T>::load(xr, q < nq ? xrow + (uint32_t)(s * C + 4 * q) * esz : kOOB, 0);
            }
            acc4 += hp[s] * xv;
        }
        // (bf16, C % 8 == 4: the upper half of the last group read the next
        // stream's columns)
        if (q >= nq) acc4 = f32x4{0.f, 0.f, 0.f, 0.f};
        v[j] = acc4;
        sq += acc4.x * acc4.x + acc4.y * acc4.y + acc4.z * acc4.z + acc4.w * acc4.w;
    }
    float scale = 1.f;
    if (a.norm_w) {
#pragma unroll
        for (int sh = 1; sh < 64; sh <<= 1) sq += __shfl_xor(sq, sh);
        scale = 1.0f / sqrtf(__fdiv_rn(sq, (float)C) + a.norm_eps);
    }
    if constexpr (sizeof(T) == 2) {
        // 8 columns per store where both halves are in the row
#pragma unroll
        for (int j = 0; j < kMaxQ; j += 2) {
            const int q = quad(j);
            if (q >= nq) continue;
            f32x4 o0 = v[j] * scale, o1 = v[j + 1] * scale;
            const uint32_t off = (uint32_t)(((int64_t)tok * a.ld_in + 4 * q) * esz);
            if (q + 1 < nq) {
                if (a.norm_w) {
                    o0 *= *(const f32x4 *)(a.norm_w + 4 * q);
                    o1 *= *(const f32x4 *)(a.norm_w + 4 * q + 4);
                }
                const u32x4 u = {pack_bf16x2(o0.x, o0.y), pack_bf16x2(o0.z, o0.w), pack_bf16x2(o1.x, o1.y),
                                 pack_bf16x2(o1.z, o1.w)};
                __builtin_amdgcn_raw_buffer_store_b128(u, lr, off, 0, 0);
            } else {
                if (a.norm_w) o0 *= *(const f32x4 *)(a.norm_w + 4 * q);
                Buf4<T>::store(o0, lr, off, 0);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < kMaxQ; ++j) {
            const int q = quad(j);
            if (q >= nq) continue;
            f32x4 o = v[j] * scale;
            if (a.norm_w) o *= *(const f32x4 *)(a.norm_w + 4 * q);
            Buf4<T>::store(o, lr, (uint32_t)(((int64_t)tok * a.ld_in + 4 * q) * esz), 0);
        }
    }
}

// The same per-token work for few tokens (decode): one 256-thread workgroup
// per token.  The split partials are summed in a fixed two-level order (8
// thread groups over strided splits, then the 8 group sums in order), the
// constraints run on lanes 0..3 as above, and the row (C <= 4096) is spread
// 16 columns per thread with the sum of squares reduced through LDS.
template <typename T>
__global__ __launch_bounds__(256) void mhc_apply_tok_kernel(ApplyArgs a) {
    constexpr uint32_t esz = sizeof(T);
    __shared__ float grp_s[8][32];
    __shared__ float dyn_s[kProjOut + 7];
    __shared__ float hpre_s[4];
    __shared__ float sq_s[4];
    __shared__ float par_s[32];  // coef[3], then bias[2n + n*n]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tok = blockIdx.x;
    const int n = a.n, C = a.C, K = n * C;
    // loads in the order they are needed (vector loads complete in order):
    // the split partials (buffer loads, zero past the splits; splits <= 64,
    // K / 256 with K <= 16384: 8 per thread), then the token's streams and the
    // norm weights, whose round trip overlaps the split sums and the
    // constraints
    const int po = tid & 31, pg = tid >> 5;
    float pv[8];
    {
        const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.part, (uint32_t)((int64_t)a.splits * a.M * kProjOut * 4));
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int sp = pg + 8 * r;
            pv[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                pr, (po < kProjOut && sp < a.splits) ? (uint32_t)((((int64_t)sp * a.M + tok) * kProjOut + po) * 4)
                                                     : kOOB,
                0, 0));
        }
    }
    const int n_par = 3 + 2 * n + n * n;
    const float par = tid < 3 ? a.coef[tid] : tid < n_par ? a.bias[tid - 3] : 0.f;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.ldx * esz));
    const __amdgpu_buffer_rsrc_t lr = make_rsrc(a.layer_in, (uint32_t)((int64_t)a.M * a.ld_in * esz));
    const uint32_t xrow = (uint32_t)((int64_t)tok * a.ldx * esz);
    const int nq = C / 4;
    constexpr int kQ = 4;  // quads per thread: 256 x 4 x 4 = 4096 columns
    f32x4 xv[kQ][kMaxStreams];
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
        const int q = tid + 256 * j;
#pragma unroll
        for (int st = 0; st < kMaxStreams; ++st)
            xv[j][st] = Buf4<T>::load(xr, (st < n && q < nq) ? xrow + (uint32_t)(st * C + 4 * q) * esz : kOOB, 0);
    }
    f32x4 nw[kQ];
    if (a.norm_w) {
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.norm_w, (uint32_t)(C * 4));
#pragma unroll
        for (int j = 0; j < kQ; ++j) {
            const int q = tid + 256 * j;
            nw[j] = Buf4<float>::load(wr, q < nq ? (uint32_t)(16 * q) : kOOB, 0);
        }
    }
    {
        // the partials added in split order
        float v = 0.f;
#pragma unroll
        for (int r = 0; r < 8; ++r) v += pv[r];
        grp_s[pg][po] = v;
    }
    if (tid < n_par) par_s[tid] = par;
    __syncthreads();
    if (tid < kProjOut) {
        float v = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) v += grp_s[g][tid];
        dyn_s[tid] = v;
    }
    __syncthreads();
    if (tid < 4) {
        const float rs = __fdiv_rn(1.0f, sqrtf(__fdiv_rn(dyn_s[kProjOut - 1], (float)K) + a.rms_eps));
        auto dynf = [&](int o) { return dyn_s[o] * rs; };
        token_constraints_quad(0, tid, tok, a.M, n, &par_s[0], &par_s[3], a.n_iter, a.sk_eps, dynf, hpre_s, a.h_pre,
                               a.h_post, a.h_res);
    }
    __syncthreads();
    float hp[kMaxStreams];
#pragma unroll
    for (int st = 0; st < kMaxStreams; ++st) hp[st] = hpre_s[st];
    f32x4 v[kQ];
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
        f32x4 acc4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < kMaxStreams; ++st)
            if (st < n) acc4 += hp[st] * xv[j][st];
        v[j] = acc4;
        sq += acc4.x * acc4.x + acc4.y * acc4.y + acc4.z * acc4.z + acc4.w * acc4.w;
    }
    float scale = 1.f;
    if (a.norm_w) {
#pragma unroll
        for (int sh = 1; sh < 64; sh <<= 1) sq += __shfl_xor(sq, sh);
        if (lane == 0) sq_s[wave] = sq;
        __syncthreads();
        sq = (sq_s[0] + sq_s[1]) + (sq_s[2] + sq_s[3]);
        scale = 1.0f / sqrtf(__fdiv_rn(sq, (float)C) + a.norm_eps);
    }
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
        const int q = tid + 256 * j;
        if (q >= nq) continue;
        f32x4 o = v[j] * scale;
        if (a.norm_w) o *= nw[j];
        Buf4<T>::store(o, lr, (uint32_t)(((int64_t)tok * a.ld_in + 4 * q) * esz), 0);
    }
}

// ---------------------------------------------------------------- post (apply)
// x_new[t, r, :] = sum_s H_res[t, r, s] x[t, s, :] + H_post[t, r] out[t, :]
template <typename T>
__global__ __launch_bounds__(256) void mhc_post_kernel(const T *__restrict__ x, int64_t ldx, const T *__restrict__ out,
                                                       int64_t ld_out, const float *__restrict__ h_res,
                                                       const float *__restrict__ h_post, T *__restrict__ x_new,
                                                       int64_t ld_new, int M, int n, int C) {
    constexpr uint32_t esz = sizeof(T);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)((int64_t)M * ldx * esz));
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(out, (uint32_t)((int64_t)M * ld_out * esz));
    const __amdgpu_buffer_rsrc_t nr = make_rsrc(x_new, (uint32_t)((int64_t)M * ld_new * esz));
    const int cq = C / 4;
    const int64_t total = (int64_t)M * cq;
    for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < total;
         item += (int64_t)gridDim.x * blockDim.x) {
        const int tok = (int)(item / cq);
        const int c = (int)(item - (int64_t)tok * cq) * 4;
        const uint32_t xo = (uint32_t)(((int64_t)tok * ldx + c) * esz);
        f32x4 xs[kMaxStreams];
#pragma unroll
        for (int s = 0; s < kMaxStreams; ++s)
            xs[s] = Buf4<T>::load(xr, s < n ? xo : kOOB, (uint32_t)(s * C) * esz);
        const f32x4 o = Buf4<T>::load(orr, (uint32_t)(((int64_t)tok * ld_out + c) * esz), 0);
        const float *hr = h_res + (int64_t)tok * n * n;
        const float *hp = h_post + (int64_t)tok * n;
        const uint32_t no = (uint32_t)(((int64_t)tok * ld_new + c) * esz);
#pragma unroll
        for (int r = 0; r < kMaxStreams; ++r) {
            if (r >= n) continue;
            f32x4 acc = hp[r] * o;
#pragma unroll
            for (int s = 0; s < kMaxStreams; ++s)
                if (s < n) acc += hr[r * n + s] * xs[s];
            Buf4<T>::store(acc, nr, no, (uint32_t)(r * C) * esz);
        }
    }
}

}  // namespace walsh

using namespace walsh;

WALSH_EXPORT int walsh_sinkhorn_fwd(const float *h, int64_t batch, int64_t n, int64_t n_iter, float eps, float *out,
                                    void *stream) {
    if (!h || !out) return set_error(WALSH_EINVAL, "walsh_sinkhorn_fwd: null pointer");
    if (batch < 0 || n < 1 || n > 8 || n_iter < 0)
        return set_error(n > 8 ? WALSH_ENOTSUP : WALSH_EINVAL,
                         "walsh_sinkhorn_fwd: batch=%lld n=%lld n_iter=%lld (n must be 1..8)", (long long)batch,
                         (long long)n, (long long)n_iter);
    if (batch == 0) return WALSH_OK;
    const int block = 128;
    int64_t grid = ceil_div(batch, block);
    if (grid > (int64_t)device_info().cu_count * 8) grid = (int64_t)device_info().cu_count * 8;
    launch(sinkhorn_kernel, dim3((unsigned)grid), dim3(block), 0, (hipStream_t)stream, h, batch, (int)n,
                       (int)n_iter, eps, out);
    return check_hip(hipGetLastError(), "walsh_sinkhorn_fwd launch");
}

WALSH_EXPORT int walsh_sinkhorn_bwd(const float *h, const float *g, int64_t batch, int64_t n, int64_t n_iter, float eps,
                                    float *dh, void *stream) {
    if (batch > 0 && (!h || !g || !dh)) return set_error(WALSH_EINVAL, "walsh_sinkhorn_bwd: null pointer");
    if (batch < 0 || n < 1 || n > 8 || n_iter < 0)
        return set_error(n > 8 ? WALSH_ENOTSUP : WALSH_EINVAL,
                         "walsh_sinkhorn_bwd: batch=%lld n=%lld n_iter=%lld (n must be 1..8)", (long long)batch,
                         (long long)n, (long long)n_iter);
    if (batch == 0) return WALSH_OK;
    const size_t lds = (size_t)n_iter * 16 * kSkBwdThreads * sizeof(float);
    if (n <= 4 && n_iter > 0 && lds <= (size_t)device_info().max_shared_per_block / 2) {
        const int64_t grid = ceil_div(batch, kSkBwdThreads);
        launch(sinkhorn_bwd_lds_kernel<4>, dim3((unsigned)grid), dim3(kSkBwdThreads), (uint32_t)lds,
               (hipStream_t)stream, h, g, batch, (int)n, (int)n_iter, eps, dh);
        return check_hip(hipGetLastError(), "walsh_sinkhorn_bwd launch");
    }
    const int block = 64;
    int64_t grid = ceil_div(batch, block);
    if (grid > (int64_t)device_info().cu_count * 16) grid = (int64_t)device_info().cu_count * 16;
    if (n <= 4)
        launch(sinkhorn_bwd_kernel<4>, dim3((unsigned)grid), dim3(block), 0, (hipStream_t)stream, h, g, batch, (int)n,
               (int)n_iter, eps, dh);
    else
        launch(sinkhorn_bwd_kernel<8>, dim3((unsigned)grid), dim3(block), 0, (hipStream_t)stream, h, g, batch, (int)n,
               (int)n_iter, eps, dh);
    return check_hip(hipGetLastError(), "walsh_sinkhorn_bwd launch");
}

WALSH_EXPORT int walsh_mhc_pre_fwd(const void *x, int64_t ldx, int64_t M, int64_t n, int64_t C, const void *phi,
                                   const float *coef, const float *bias, float rms_eps, int64_t n_iter, float sk_eps,
                                   float *h_pre, float *h_post, float *h_res, void *layer_in, int64_t ld_in,
                                   int dtype, void *stream) {
    if (!x || !phi || !coef || !bias || !h_pre || !h_post || !h_res || !layer_in)
        return set_error(WALSH_EINVAL, "walsh_mhc_pre_fwd: null pointer");
    if (M < 0 || n < 1 || C < 4 || ldx < n * C || ld_in < C || n_iter < 0)
        return set_error(WALSH_EINVAL, "walsh_mhc_pre_fwd: bad shape M=%lld n=%lld C=%lld", (long long)M,
                         (long long)n, (long long)C);
    if (n > kMaxStreams || C % 4 != 0 || ldx % 4 != 0 || ld_in % 4 != 0)
        return set_error(WALSH_ENOTSUP, "walsh_mhc_pre_fwd: needs n <= %d and C, row strides multiples of 4",
                         kMaxStreams);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16)
        return set_error(WALSH_ENOTSUP, "walsh_mhc_pre_fwd: dtype %d", dtype);
    if (M == 0) return WALSH_OK;
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4;
    const size_t valign = dtype == WALSH_BF16 ? 8 : 16;
    if ((uintptr_t)x % valign || (uintptr_t)layer_in % valign || (uintptr_t)phi % valign)
        return set_error(WALSH_ENOTSUP, "walsh_mhc_pre_fwd: x, phi and layer_in must be %zu-byte aligned", valign);
    if ((int64_t)kPhiRows * n * C * esz > (int64_t)kMaxBufferBytes)
        return set_error(WALSH_ENOTSUP, "walsh_mhc_pre_fwd: projection too large");
    const int64_t ld = ldx > ld_in ? ldx : ld_in;
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * esz) / kPreTok * kPreTok;
    if (rows_max < kPreTok) return set_error(WALSH_ENOTSUP, "walsh_mhc_pre_fwd: row stride too large");
    rows_max = balanced_rows(M, rows_max, kPreTok);
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        PreArgs a;
        a.x = (const char *)x + r0 * ldx * esz;
        a.ldx = ldx;
        a.M = (int)rows;
        a.n = (int)n;
        a.C = (int)C;
        a.phi = phi;
        a.coef = coef;
        a.bias = bias;
        a.rms_eps = rms_eps;
        a.sk_eps = sk_eps;
        a.n_iter = (int)n_iter;
        a.h_pre = h_pre + r0 * n;
        a.h_post = h_post + r0 * n;
        a.h_res = h_res + r0 * n * n;
        a.layer_in = (char *)layer_in + r0 * ld_in * esz;
        a.ld_in = ld_in;
        const dim3 G((unsigned)ceil_div(rows, kPreTok)), B(kPreThreads);
        if (dtype == WALSH_BF16)
            launch((mhc_pre_kernel<uint16_t, true>), G, B, 0, (hipStream_t)stream, a);
        else
            launch((mhc_pre_kernel<float, false>), G, B, 0, (hipStream_t)stream, a);
        const int rc = check_hip(hipGetLastError(), "walsh_mhc_pre_fwd launch");
        if (rc) return rc;
    }
    return WALSH_OK;
}

WALSH_EXPORT int walsh_mhc_post_fwd(const void *x, int64_t ldx, const void *out, int64_t ld_out, const float *h_res,
                                    const float *h_post, void *x_new, int64_t ld_new, int64_t M, int64_t n, int64_t C,
                                    int dtype, void *stream) {
    if (!x || !out || !h_res || !h_post || !x_new) return set_error(WALSH_EINVAL, "walsh_mhc_post_fwd: null pointer");
    if (M < 0 || n < 1 || C < 4 || ldx < n * C || ld_new < n * C || ld_out < C)
        return set_error(WALSH_EINVAL, "walsh_mhc_post_fwd: bad shape M=%lld n=%lld C=%lld", (long long)M,
                         (long long)n, (long long)C);
    if (n > kMaxStreams || C % 4 || ldx % 4 || ld_out % 4 || ld_new % 4)
        return set_error(WALSH_ENOTSUP, "walsh_mhc_post_fwd: needs n <= %d and C, row strides multiples of 4",
                         kMaxStreams);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "walsh_mhc_post_fwd: dtype");
    if (M == 0) return WALSH_OK;
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4;
    const size_t valign = dtype == WALSH_BF16 ? 8 : 16;
    if ((uintptr_t)x % valign || (uintptr_t)out % valign || (uintptr_t)x_new % valign)
        return set_error(WALSH_ENOTSUP, "walsh_mhc_post_fwd: tensors must be %zu-byte aligned", valign);
    int64_t ld = ldx > ld_new ? ldx : ld_new;
    if (ld_out > ld) ld = ld_out;
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * esz);
    if (rows_max < 1) return set_error(WALSH_ENOTSUP, "walsh_mhc_post_fwd: row stride too large");
    rows_max = balanced_rows(M, rows_max, 1);
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        const int block = 256;
        int64_t grid = ceil_div(rows * (C / 4), block);
        const int64_t cap = (int64_t)device_info().cu_count * 8;
        if (grid > cap) grid = cap;
        hipStream_t s = (hipStream_t)stream;
        if (dtype == WALSH_BF16)
            launch(mhc_post_kernel<uint16_t>, dim3((unsigned)grid), dim3(block), 0, s,
                               (const uint16_t *)x + r0 * ldx, ldx, (const uint16_t *)out + r0 * ld_out, ld_out,
                               h_res + r0 * n * n, h_post + r0 * n, (uint16_t *)x_new + r0 * ld_new, ld_new, (int)rows,
                               (int)n, (int)C);
        else
            launch(mhc_post_kernel<float>, dim3((unsigned)grid), dim3(block), 0, s,
                               (const float *)x + r0 * ldx, ldx, (const float *)out + r0 * ld_out, ld_out,
                               h_res + r0 * n * n, h_post + r0 * n, (float *)x_new + r0 * ld_new, ld_new, (int)rows,
                               (int)n, (int)C);
        const int rc = check_hip(hipGetLastError(), "walsh_mhc_post_fwd launch");
        if (rc) return rc;
    }
    return WALSH_OK;
}

struct PostIn {
    const void *xo;
    int64_t ld_xo;
    const void *out;
    int64_t ld_out;
    const float *hr_prev, *hp_prev;
    void *x_new;
    int64_t ld_new;
};

static int mhc_pre_norm_impl(const char *fn, const void *x, int64_t ldx, int64_t M, int64_t n, int64_t C,
                             const void *phi_frag, const float *coef, const float *bias, float rms_eps, int64_t n_iter,
                             float sk_eps, float *h_pre, float *h_post, float *h_res, void *layer_in, int64_t ld_in,
                             const float *norm_w, float norm_eps, int dtype, void *stream, const PostIn *post) {
    if ((!post && !x) || !phi_frag || !coef || !bias || !h_pre || !h_post || !h_res || !layer_in)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || n < 1 || C < 4 || (!post && ldx < n * C) || ld_in < C || n_iter < 0)
        return set_error(WALSH_EINVAL, "%s: bad shape M=%lld n=%lld C=%lld", fn, (long long)M, (long long)n,
                         (long long)C);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype", fn);
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4;
    const int64_t rowb = n * C * esz;
    if (n > kMaxStreams || (n * C) % 16 || C % 4 || C > 1024 || rowb % 16 || (!post && ldx % (16 / esz)) ||
        ld_in % 4 || rowb * 16 > kTileBytes)
        return set_error(WALSH_ENOTSUP, "%s: needs n <= %d, n*C %% 16 == 0, C <= 1024, 16 rows in 128 KB", fn,
                         kMaxStreams);
    if ((!post && (uintptr_t)x % 16) || (uintptr_t)layer_in % 16 || (uintptr_t)phi_frag % 16 ||
        (norm_w && (uintptr_t)norm_w % 16))
        return set_error(WALSH_ENOTSUP, "%s: pointers must be 16-byte aligned", fn);
    if (post) {
        if (!post->xo || !post->out || !post->hr_prev || !post->hp_prev || !post->x_new)
            return set_error(WALSH_EINVAL, "%s: null pointer", fn);
        const int64_t v = 16 / esz;
        if ((C * esz) % 16 || post->ld_xo < n * C || post->ld_new < n * C || post->ld_out < C || post->ld_xo % v ||
            post->ld_new % v || post->ld_out % v || (uintptr_t)post->xo % 16 || (uintptr_t)post->out % 16 ||
            (uintptr_t)post->x_new % 16)
            return set_error(WALSH_ENOTSUP, "%s: stream rows need C*esize %% 16 == 0, 16-byte aligned rows", fn);
        if (post->x_new == post->xo || (const float *)post->hr_prev == h_res || (const float *)post->hp_prev == h_post)
            return set_error(WALSH_EINVAL, "%s: outputs may not alias the previous stream's tensors", fn);
    }
    if (M == 0) return WALSH_OK;
    // 16-token tiles: ~74 KB of LDS at 4 KB rows, so two workgroups share a
    // CU and overlap their load / projection / write phases
    const int MT = 1;
    const int TT = 16 * MT;
    const size_t lds = (size_t)TT * (rowb + 8) + (size_t)kPreWaves * TT * (kPhiRows + 1) * 4 + kPreWaves * TT * 4 +
                       TT * 16 + (size_t)C * 4 + 32 * 4;   // ... norm weights, coef and bias
    if (lds > (size_t)device_info().max_shared_per_block)
        return set_error(WALSH_ENOTSUP, "%s: needs %zu B of LDS", fn, lds);
    int64_t ld = ld_in;
    if (!post && ldx > ld) ld = ldx;
    if (post) {
        if (post->ld_xo > ld) ld = post->ld_xo;
        if (post->ld_new > ld) ld = post->ld_new;
        if (post->ld_out > ld) ld = post->ld_out;
    }
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * esz) / TT * TT;
    if (rows_max < TT) return set_error(WALSH_ENOTSUP, "%s: row stride too large", fn);
    rows_max = balanced_rows(M, rows_max, TT);
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        Pre2Args a{};
        a.x = post ? nullptr : (const char *)x + r0 * ldx * esz;
        a.ldx = ldx;
        a.M = (int)rows;
        a.n = (int)n;
        a.C = (int)C;
        a.phi_frag = phi_frag;
        a.coef = coef;
        a.bias = bias;
        a.rms_eps = rms_eps;
        a.sk_eps = sk_eps;
        a.n_iter = (int)n_iter;
        a.h_pre = h_pre + r0 * n;
        a.h_post = h_post + r0 * n;
        a.h_res = h_res + r0 * n * n;
        a.layer_in = (char *)layer_in + r0 * ld_in * esz;
        a.ld_in = ld_in;
        a.norm_w = norm_w;
        a.norm_eps = norm_eps;
        if (post) {
            a.xo = (const char *)post->xo + r0 * post->ld_xo * esz;
            a.ld_xo = post->ld_xo;
            a.out = (const char *)post->out + r0 * post->ld_out * esz;
            a.ld_out = post->ld_out;
            a.hr_prev = post->hr_prev + r0 * n * n;
            a.hp_prev = post->hp_prev + r0 * n;
            a.x_new = (char *)post->x_new + r0 * post->ld_new * esz;
            a.ld_new = post->ld_new;
        }
        const dim3 G((unsigned)ceil_div(rows, TT)), B(kPreThreads);
        hipStream_t s = (hipStream_t)stream;
        const bool fast = n == 4 && C == 512;
        if (dtype == WALSH_BF16) {
            if (post && fast) launch((mhc_pre2_kernel<uint16_t, true, 1, true, true>), G, B, lds, s, a);
            else if (post) launch((mhc_pre2_kernel<uint16_t, true, 1, true>), G, B, lds, s, a);
            else if (fast) launch((mhc_pre2_kernel<uint16_t, true, 1, false, true>), G, B, lds, s, a);
            else launch((mhc_pre2_kernel<uint16_t, true, 1>), G, B, lds, s, a);
        } else {
            if (post && fast) launch((mhc_pre2_kernel<float, false, 1, true, true>), G, B, lds, s, a);
            else if (post) launch((mhc_pre2_kernel<float, false, 1, true>), G, B, lds, s, a);
            else if (fast) launch((mhc_pre2_kernel<float, false, 1, false, true>), G, B, lds, s, a);
            else launch((mhc_pre2_kernel<float, false, 1>), G, B, lds, s, a);
        }
        const int rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
    }
    return WALSH_OK;
}

WALSH_EXPORT int walsh_mhc_pre_norm_fwd(const void *x, int64_t ldx, int64_t M, int64_t n, int64_t C,
                                        const void *phi_frag, const float *coef, const float *bias, float rms_eps,
                                        int64_t n_iter, float sk_eps, float *h_pre, float *h_post, float *h_res,
                                        void *layer_in, int64_t ld_in, const float *norm_w, float norm_eps,
                                        int dtype, void *stream) {
    return mhc_pre_norm_impl("walsh_mhc_pre_norm_fwd", x, ldx, M, n, C, phi_frag, coef, bias, rms_eps, n_iter, sk_eps,
                             h_pre, h_post, h_res, layer_in, ld_in, norm_w, norm_eps, dtype, stream, nullptr);
}

WALSH_EXPORT int walsh_mhc_post_pre_norm_fwd(const void *x_old, int64_t ld_old, const void *out, int64_t ld_out,
                                             const float *h_res_prev, const float *h_post_prev, void *x_new,
                                             int64_t ld_new, int64_t M, int64_t n, int64_t C, const void *phi_frag,
                                             const float *coef, const float *bias, float rms_eps, int64_t n_iter,
                                             float sk_eps, float *h_pre, float *h_post, float *h_res, void *layer_in,
                                             int64_t ld_in, const float *norm_w, float norm_eps, int dtype,
                                             void *stream) {
    const PostIn post{x_old, ld_old, out, ld_out, h_res_prev, h_post_prev, x_new, ld_new};
    return mhc_pre_norm_impl("walsh_mhc_post_pre_norm_fwd", nullptr, 0, M, n, C, phi_frag, coef, bias, rms_eps,
                             n_iter, sk_eps, h_pre, h_post, h_res, layer_in, ld_in, norm_w, norm_eps, dtype, stream,
                             &post);
}

// Splits of K for the wide-row projection: enough wavefronts to fill the
// chip when there are few tokens (decode), one split otherwise.
// row counts up to which the apply step runs a workgroup per token
constexpr int64_t kApplyTokRows = 1024;

static int mhc_wide_splits(int64_t M, int64_t K) {
    const int64_t tiles = ceil_div(M, 16);
    const int64_t want = (int64_t)device_info().cu_count * 8;
    int64_t s = tiles >= want ? 1 : ceil_div(want, tiles);
    const int64_t smax = K / 256;             // at least 256 columns per split
    if (s > smax) s = smax;
    return (int)(s < 1 ? 1 : s);
}

WALSH_EXPORT int64_t walsh_mhc_pre_wide_workspace(int64_t M, int64_t n, int64_t C) {
    if (M < 0 || n < 1 || C < 1) return 0;
    return (int64_t)mhc_wide_splits(M, n * C) * M * kProjOut * 4;
}

// The per-token apply launch of the wide mapping on rows [r0, r0 + rows)
// (x already offset to row r0), after a projection wrote its partial sums.
static void wide_apply_launch(const void *xc, int64_t ldx, int64_t rows, int64_t r0, int64_t n, int64_t C,
                              int splits, const float *part, const float *coef, const float *bias, float rms_eps,
                              int64_t n_iter, float sk_eps, float *h_pre, float *h_post, float *h_res, void *layer_in,
                              int64_t ld_in, const float *norm_w, float norm_eps, int dtype, hipStream_t s) {
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4;
    ApplyArgs aa;
    aa.x = xc;
    aa.ldx = ldx;
    aa.M = (int)rows;
    aa.n = (int)n;
    aa.C = (int)C;
    aa.splits = splits;
    aa.part = part;
    aa.coef = coef;
    aa.bias = bias;
    aa.rms_eps = rms_eps;
    aa.sk_eps = sk_eps;
    aa.n_iter = (int)n_iter;
    aa.h_pre = h_pre + r0 * n;
    aa.h_post = h_post + r0 * n;
    aa.h_res = h_res + r0 * n * n;
    aa.layer_in = (char *)layer_in + r0 * ld_in * esz;
    aa.ld_in = ld_in;
    aa.norm_w = norm_w;
    aa.norm_eps = norm_eps;
    const dim3 B(256);
    if (rows <= kApplyTokRows && splits <= 64) {
        // few tokens: a workgroup per token
        const dim3 G2((unsigned)rows);
        if (dtype == WALSH_BF16) launch(mhc_apply_tok_kernel<uint16_t>, G2, B, 0, s, aa);
        else launch(mhc_apply_tok_kernel<float>, G2, B, 0, s, aa);
    } else {
        const dim3 G2((unsigned)ceil_div(rows, 4));
        if (dtype == WALSH_BF16) launch(mhc_apply_kernel<uint16_t>, G2, B, 0, s, aa);
        else launch(mhc_apply_kernel<float>, G2, B, 0, s, aa);
    }
}

WALSH_EXPORT int walsh_mhc_pre_wide_fwd(const void *x, int64_t ldx, int64_t M, int64_t n, int64_t C,
                                        const void *phi_frag32, const float *coef, const float *bias, float rms_eps,
                                        int64_t n_iter, float sk_eps, float *h_pre, float *h_post, float *h_res,
                                        void *layer_in, int64_t ld_in, const float *norm_w, float norm_eps,
                                        void *workspace, int64_t workspace_bytes, int dtype, void *stream) {
    const char *fn = "walsh_mhc_pre_wide_fwd";
    if (!x || !phi_frag32 || !coef || !bias || !h_pre || !h_post || !h_res || !layer_in)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || n < 1 || C < 4 || ldx < n * C || ld_in < C || n_iter < 0)
        return set_error(WALSH_EINVAL, "%s: bad shape M=%lld n=%lld C=%lld", fn, (long long)M, (long long)n,
                         (long long)C);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype", fn);
    const int64_t esz = dtype == WALSH_BF16 ? 2 : 4, K = n * C;
    if (n > kMaxStreams || K % 32 || C % 4 || C > 4096 || ldx % (32 / esz) || ld_in % 4)
        return set_error(WALSH_ENOTSUP, "%s: needs n <= %d, n*C %% 32 == 0, C <= 4096", fn, kMaxStreams);
    if ((uintptr_t)x % 16 || (uintptr_t)layer_in % 16 || (uintptr_t)phi_frag32 % 16 ||
        (norm_w && (uintptr_t)norm_w % 16))
        return set_error(WALSH_ENOTSUP, "%s: pointers must be 16-byte aligned", fn);
    if (M == 0) return WALSH_OK;
    const int splits = mhc_wide_splits(M, K);
    // the per-token launches hold one split per lane
    if (splits > 64) return set_error(WALSH_ENOTSUP, "%s: %d K splits (at most 64)", fn, splits);
    const int64_t need = (int64_t)splits * M * kProjOut * 4;
    if (!workspace || workspace_bytes < need)
        return set_error(WALSH_EINVAL, "%s: workspace of %lld bytes needed", fn, (long long)need);
    // row chunks keep every buffer below 2^31 bytes
    const int64_t ld = ldx > ld_in ? ldx : ld_in;
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * esz) / 16 * 16;
    if (rows_max < 16) return set_error(WALSH_ENOTSUP, "%s: row stride too large", fn);
    rows_max = balanced_rows(M, rows_max, 16);
    hipStream_t s = (hipStream_t)stream;
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        const void *xc = (const char *)x + r0 * ldx * esz;
        ProjArgs pa;
        pa.x = xc;
        pa.ldx = ldx;
        pa.M = (int)rows;
        pa.K = (int)K;
        pa.splits = splits;
        pa.kper = (int)(ceil_div(ceil_div(K, splits), 32) * 32);
        pa.phi32 = phi_frag32;
        pa.part = (float *)workspace;
        const int64_t items = ceil_div(rows, 16) * splits;
        const dim3 G1((unsigned)ceil_div(items, 4)), B(256);
        if (dtype == WALSH_BF16) launch(mhc_proj_kernel<uint16_t>, G1, B, 0, s, pa);
        else launch(mhc_proj_kernel<float>, G1, B, 0, s, pa);
        wide_apply_launch(xc, ldx, rows, r0, n, C, splits, (const float *)workspace, coef, bias, rms_eps, n_iter,
                          sk_eps, h_pre, h_post, h_res, layer_in, ld_in, norm_w, norm_eps, dtype, s);
        const int rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
    }
    return WALSH_OK;
}

WALSH_EXPORT int walsh_mhc_post_pre_wide_fwd(const void *xo, int64_t ld_xo, const void *out, int64_t ld_out,
                                             const float *hr_prev, const float *hp_prev, void *x_new, int64_t ld_new,
                                             int64_t M, int64_t n, int64_t C, const void *phi_frag32,
                                             const float *coef, const float *bias, float rms_eps, int64_t n_iter,
                                             float sk_eps, float *h_pre, float *h_post, float *h_res, void *layer_in,
                                             int64_t ld_in, const float *norm_w, float norm_eps, void *workspace,
                                             int64_t workspace_bytes, int dtype, void *stream) {
    const char *fn = "walsh_mhc_post_pre_wide_fwd";
    if (!xo || !out || !hr_prev || !hp_prev || !x_new || !phi_frag32 || !coef || !bias || !h_pre || !h_post ||
        !h_res || !layer_in)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (M < 0 || n < 1 || C < 32 || ld_xo < n * C || ld_new < n * C || ld_out < C || ld_in < C || n_iter < 0)
        return set_error(WALSH_EINVAL, "%s: bad shape M=%lld n=%lld C=%lld", fn, (long long)M, (long long)n,
                         (long long)C);
    if (dtype != WALSH_BF16 || n > kMaxStreams || C % 32 || C > 4096 || ld_xo % 8 || ld_new % 8 || ld_out % 8 ||
        ld_in % 4)
        return set_error(WALSH_ENOTSUP, "%s: needs bf16, n <= %d, C a multiple of 32 up to 4096, row strides "
                         "multiples of 8", fn, kMaxStreams);
    if ((uintptr_t)xo % 16 || (uintptr_t)out % 16 || (uintptr_t)x_new % 16 || (uintptr_t)layer_in % 16 ||
        (uintptr_t)phi_frag32 % 16 || (norm_w && (uintptr_t)norm_w % 16))
        return set_error(WALSH_ENOTSUP, "%s: pointers must be 16-byte aligned", fn);
    if (M == 0) return WALSH_OK;
    const int64_t K = n * C;
    const int splits = mhc_wide_splits(M, K);
    // the per-token launches hold one split per lane
    if (splits > 64) return set_error(WALSH_ENOTSUP, "%s: %d K splits (at most 64)", fn, splits);
    const int64_t need = (int64_t)splits * M * kProjOut * 4;
    if (!workspace || workspace_bytes < need)
        return set_error(WALSH_EINVAL, "%s: workspace of %lld bytes needed", fn, (long long)need);
    int64_t ld = ld_xo > ld_new ? ld_xo : ld_new;
    if (ld_in > ld) ld = ld_in;
    int64_t rows_max = (int64_t)kMaxBufferBytes / (ld * 2) / 16 * 16;
    if (rows_max < 16) return set_error(WALSH_ENOTSUP, "%s: row stride too large", fn);
    rows_max = balanced_rows(M, rows_max, 16);
    hipStream_t s = (hipStream_t)stream;
    for (int64_t r0 = 0; r0 < M; r0 += rows_max) {
        const int64_t rows = (M - r0) < rows_max ? (M - r0) : rows_max;
        PostProjArgs pa;
        pa.xo = (const uint16_t *)xo + r0 * ld_xo;
        pa.ld_xo = ld_xo;
        pa.out = (const uint16_t *)out + r0 * ld_out;
        pa.ld_out = ld_out;
        pa.hr_prev = hr_prev + r0 * n * n;
        pa.hp_prev = hp_prev + r0 * n;
        pa.x_new = (uint16_t *)x_new + r0 * ld_new;
        pa.ld_new = ld_new;
        pa.M = (int)rows;
        pa.n = (int)n;
        pa.C = (int)C;
        pa.splits = splits;
        pa.cper = (int)(ceil_div(ceil_div(C, splits), 32) * 32);
        pa.phi32 = (const uint16_t *)phi_frag32;
        pa.part = (float *)workspace;
        const int64_t items = ceil_div(rows, 16) * splits;
        const dim3 G((unsigned)ceil_div(items, 4)), B(256);
        switch (n) {
        case 1: launch(mhc_post_proj_kernel<1>, G, B, 0, s, pa); break;
        case 2: launch(mhc_post_proj_kernel<2>, G, B, 0, s, pa); break;
        case 3: launch(mhc_post_proj_kernel<3>, G, B, 0, s, pa); break;
        default: launch(mhc_post_proj_kernel<4>, G, B, 0, s, pa); break;
        }
        wide_apply_launch(pa.x_new, ld_new, rows, r0, n, C, splits, (const float *)workspace, coef, bias, rms_eps,
                          n_iter, sk_eps, h_pre, h_post, h_res, layer_in, ld_in, norm_w, norm_eps, dtype, s);
        const int rc = check_hip(hipGetLastError(), fn);
        if (rc) return rc;
    }
    return WALSH_OK;
}

static int mix_check(const char *fn, int64_t M, int64_t n, int64_t C, int dtype) {
    if (M < 0 || n < 1 || n > kMaxStreams || C < 4 || C % 4)
        return set_error(WALSH_EINVAL, "%s: bad shape M=%lld n=%lld C=%lld (n <= %d, C a multiple of 4)", fn,
                         (long long)M, (long long)n, (long long)C, kMaxStreams);
    if (dtype != WALSH_F32 && dtype != WALSH_BF16) return set_error(WALSH_ENOTSUP, "%s: dtype %d", fn, dtype);
    return WALSH_OK;
}

static dim3 mix_grid(int64_t M) {
    int64_t g = ceil_div(M, kMixWaves);
    const int64_t cap = (int64_t)device_info().cu_count * 16;
    return dim3((unsigned)(g < cap ? g : cap));
}

WALSH_EXPORT int walsh_mhc_aggregate_fwd(const void *x, const float *h_pre, void *layer_in, int64_t M, int64_t n,
                                         int64_t C, int dtype, void *stream) {
    const char *fn = "walsh_mhc_aggregate_fwd";
    int rc = mix_check(fn, M, n, C, dtype);
    if (rc) return rc;
    if (M == 0) return WALSH_OK;
    if (!x || !h_pre || !layer_in) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (dtype == WALSH_BF16)
        launch(mhc_agg_fwd_kernel<uint16_t>, mix_grid(M), dim3(64 * kMixWaves), 0, (hipStream_t)stream,
               (const uint16_t *)x, h_pre, (uint16_t *)layer_in, M, (int)n, (int)C);
    else
        launch(mhc_agg_fwd_kernel<float>, mix_grid(M), dim3(64 * kMixWaves), 0, (hipStream_t)stream, (const float *)x,
               h_pre, (float *)layer_in, M, (int)n, (int)C);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_mhc_aggregate_bwd(const void *x, const float *h_pre, const void *d_layer_in, void *dx,
                                         float *dh_pre, int64_t M, int64_t n, int64_t C, int dtype, void *stream) {
    const char *fn = "walsh_mhc_aggregate_bwd";
    int rc = mix_check(fn, M, n, C, dtype);
    if (rc) return rc;
    if (M == 0) return WALSH_OK;
    if (!x || !h_pre || !d_layer_in || !dx || !dh_pre) return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (dtype == WALSH_BF16)
        launch(mhc_agg_bwd_kernel<uint16_t>, mix_grid(M), dim3(64 * kMixWaves), 0, (hipStream_t)stream,
               (const uint16_t *)x, h_pre, (const uint16_t *)d_layer_in, (uint16_t *)dx, dh_pre, M, (int)n, (int)C);
    else
        launch(mhc_agg_bwd_kernel<float>, mix_grid(M), dim3(64 * kMixWaves), 0, (hipStream_t)stream, (const float *)x,
               h_pre, (const float *)d_layer_in, (float *)dx, dh_pre, M, (int)n, (int)C);
    return check_hip(hipGetLastError(), fn);
}

WALSH_EXPORT int walsh_mhc_post_bwd(const void *x, const void *out, const float *h_res, const float *h_post,
                                    const void *d_new, void *dx, void *d_out, float *dh_res, float *dh_post, int64_t M,
                                    int64_t n, int64_t C, int dtype, void *stream) {
    const char *fn = "walsh_mhc_post_bwd";
    int rc = mix_check(fn, M, n, C, dtype);
    if (rc) return rc;
    if (M == 0) return WALSH_OK;
    if (!x || !out || !h_res || !h_post || !d_new || !dx || !d_out || !dh_res || !dh_post)
        return set_error(WALSH_EINVAL, "%s: null pointer", fn);
    if (dtype == WALSH_BF16)
        launch(mhc_post_bwd_kernel<uint16_t>, mix_grid(M), dim3(64 * kMixWaves), 0, (hipStream_t)stream,
               (const uint16_t *)x, (const uint16_t *)out, h_res, h_post, (const uint16_t *)d_new, (uint16_t *)dx,
               (uint16_t *)d_out, dh_res, dh_post, M, (int)n, (int)C);
    else
        launch(mhc_post_bwd_kernel<float>, mix_grid(M), dim3(64 * kMixWaves), 0, (hipStream_t)stream, (const float *)x,
               (const float *)out, h_res, h_post, (const float *)d_new, (float *)dx, (float *)d_out, dh_res, dh_post,
               M, (int)n, (int)C);
    return check_hip(hipGetLastError(), fn);
}
