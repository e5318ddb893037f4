// Shared helpers for the Walsh HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "walsh.h"

#define WALSH_EXPORT extern "C" __attribute__((visibility("default")))

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

namespace walsh {

// ---------------------------------------------------------------- errors
// Thread-local message behind walsh_last_error(); set_error returns the code.
int set_error(int code, const char *fmt, ...);
int check_hip(hipError_t e, const char *what);

// Launch-time device facts (queried once per device, cached).
struct DeviceInfo {
    int cu_count;
    int max_shared_per_block;
    int lds_per_cu;  // LDS bytes of one CU (160 KB on gfx950), shared by its resident workgroups
};
const DeviceInfo &device_info();

// ---------------------------------------------------------------- timing
// Optional per-launch timing (walsh_timing_begin / _end): while it is on,
// every launch records the kernel's own start and stop timestamps
// (hipExtLaunchKernelGGL) into the next event pair of a pool, labelled with
// the tag the caller set last.  Not thread-safe while on.
struct Timing {
    bool on;
    int tag, n, cap;
    hipEvent_t *ev;  // 2 * cap events
    int *tags;       // cap
};
Timing &timing();

template <typename F, typename... Args>
inline void launch(F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Args... args) {
    Timing &t = timing();
    if (t.on && t.n < t.cap) {
        hipExtLaunchKernelGGL(kernel, grid, block, lds, s, t.ev[2 * t.n], t.ev[2 * t.n + 1], 0, args...);
        t.tags[t.n++] = t.tag;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
    }
}

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}
// Round-to-nearest-even float -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r;
    r.x = (__bf16)lo;
    r.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    __bf16 r = (__bf16)v;
    return __builtin_bit_cast(uint16_t, r);
}

// Element access for the two activation types.
template <typename T> struct Act;
template <> struct Act<float> {
    static __device__ __forceinline__ float load(const float *p) { return *p; }
    static __device__ __forceinline__ void store(float *p, float v) { *p = v; }
};
template <> struct Act<uint16_t> {
    static __device__ __forceinline__ float load(const uint16_t *p) { return bf16_to_f32(*p); }
    static __device__ __forceinline__ void store(uint16_t *p, float v) { *p = f32_to_bf16(v); }
};

// 4 consecutive activations <-> float4 (requires 16-byte (f32) / 8-byte (bf16) alignment).
__device__ __forceinline__ f32x4 load4(const float *p) { return *(const f32x4 *)p; }
__device__ __forceinline__ f32x4 load4(const uint16_t *p) {
    uint2 u = *(const uint2 *)p;
    f32x4 r;
    r.x = __uint_as_float(u.x << 16);
    r.y = __uint_as_float(u.x & 0xffff0000u);
    r.z = __uint_as_float(u.y << 16);
    r.w = __uint_as_float(u.y & 0xffff0000u);
    return r;
}
__device__ __forceinline__ void store4(float *p, f32x4 v) { *(f32x4 *)p = v; }
__device__ __forceinline__ void store4(uint16_t *p, f32x4 v) {
    uint2 u;
    u.x = pack_bf16x2(v.x, v.y);
    u.y = pack_bf16x2(v.z, v.w);
    *(uint2 *)p = u;
}

// Workgroup barrier ordering LDS only: global loads and stores issued before
// it stay in flight instead of being drained at every phase boundary (as the
// full __syncthreads() fence does).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Ordering of LDS accesses between the lanes of one wavefront: a wave's LDS
// instructions execute in order, so this only stops the compiler from moving
// accesses across it (no wait, no barrier instruction).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Rows per launch when M rows must be split into launches of at most
// rows_max (a multiple of align): equal chunks rounded up to align, so no
// launch is a small tail.
inline int64_t balanced_rows(int64_t M, int64_t rows_max, int64_t align) {
    if (M <= rows_max) return rows_max;
    const int64_t n = ceil_div(M, rows_max);
    const int64_t r = ceil_div(ceil_div(M, n), align) * align;
    return r < rows_max ? r : rows_max;
}

// ---------------------------------------------------------------- buffer access
// Raw buffer resources (gfx9 descriptor word 3 = 0x00020000).  A lane whose
// byte offset is >= the buffer size reads zeros and its stores are dropped,
// which replaces per-lane branches for tails.  kOOB is such an offset.
constexpr uint32_t kOOB = 0x80000000u;
constexpr uint32_t kMaxBufferBytes = 0x7fffffffu;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// 4 activations at byte offset voff + soff (8 bytes for bf16, 16 for f32).
template <typename T> struct Buf4;
template <> struct Buf4<float> {
    static __device__ __forceinline__ f32x4 load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    }
    static __device__ __forceinline__ void store(f32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff, soff, 0);
    }
    static __device__ __forceinline__ float load1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
    }
    static __device__ __forceinline__ void store1(float v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff, soff, 0);
    }
};
template <> struct Buf4<uint16_t> {
    static __device__ __forceinline__ f32x4 load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
        const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
        f32x4 v;
        v.x = __uint_as_float(u.x << 16);
        v.y = __uint_as_float(u.x & 0xffff0000u);
        v.z = __uint_as_float(u.y << 16);
        v.w = __uint_as_float(u.y & 0xffff0000u);
        return v;
    }
    static __device__ __forceinline__ void store(f32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
        u32x2 u;
        u.x = pack_bf16x2(v.x, v.y);
        u.y = pack_bf16x2(v.z, v.w);
        __builtin_amdgcn_raw_buffer_store_b64(u, r, voff, soff, 0);
    }
    static __device__ __forceinline__ float load1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
        const uint16_t b = __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
        return bf16_to_f32(b);
    }
    static __device__ __forceinline__ void store1(float v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, f32_to_bf16(v)), r, voff, soff, 0);
    }
};

}  // namespace walsh
