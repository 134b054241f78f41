// Device-side building blocks for the gfx950 (CDNA4, wave64) kernels of
// libt2h: 16-byte packs of f32/f16/bf16 storage with f32 math, DPP row and
// wave reductions, and the token-row -> batch map.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "t2h.h"

namespace t2h {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// storage types
// ---------------------------------------------------------------------------
template <int DT> struct Storage;
template <> struct Storage<T2H_F32> { using type = float; };
template <> struct Storage<T2H_F16> { using type = _Float16; };
template <> struct Storage<T2H_BF16> { using type = __bf16; };

template <typename T> constexpr int kPack = 16 / (int)sizeof(T);  // elements per 16 B

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) {
    return __builtin_bit_cast(float, b16 << 16);
}

// f32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (u >> 16) | 0x40u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);  // RNE
}

// Unpack / pack one 32-bit word holding 32/(8*sizeof(T)) elements.
template <typename T> struct Word;
template <> struct Word<float> {
    static constexpr int N = 1;
    __device__ static __forceinline__ void unpack(uint32_t w, float* f) { f[0] = __builtin_bit_cast(float, w); }
    __device__ static __forceinline__ uint32_t pack(const float* f) { return __builtin_bit_cast(uint32_t, f[0]); }
};
template <> struct Word<_Float16> {
    static constexpr int N = 2;
    __device__ static __forceinline__ void unpack(uint32_t w, float* f) {
        f[0] = f16_bits_to_f32(w & 0xFFFFu);
        f[1] = f16_bits_to_f32(w >> 16);
    }
    __device__ static __forceinline__ uint32_t pack(const float* f) {
        return f32_to_f16_bits(f[0]) | (f32_to_f16_bits(f[1]) << 16);
    }
};
template <> struct Word<__bf16> {
    static constexpr int N = 2;
    __device__ static __forceinline__ void unpack(uint32_t w, float* f) {
        f[0] = __builtin_bit_cast(float, w << 16);
        f[1] = __builtin_bit_cast(float, w & 0xFFFF0000u);
    }
    __device__ static __forceinline__ uint32_t pack(const float* f) {
        return f32_to_bf16_bits(f[0]) | (f32_to_bf16_bits(f[1]) << 16);
    }
};

#ifndef T2H_NT
#define T2H_NT 1
#endif

// Load / store E contiguous elements of T as f32 (E * sizeof(T) is a multiple
// of 8 bytes; 16-byte pieces where possible). NT = non-temporal hint for data
// that is streamed once.
template <typename T, int E, bool NT_ = false>
__device__ __forceinline__ void load_elems(const T* __restrict__ p, float* f) {
    constexpr bool NT = NT_ && T2H_NT;
    constexpr int BYTES = E * (int)sizeof(T);
    static_assert(BYTES % 8 == 0, "vector width");
    constexpr int WN = Word<T>::N;
    if constexpr (BYTES % 16 == 0) {
        const u32x4* q = reinterpret_cast<const u32x4*>(p);
#pragma unroll
        for (int c = 0; c < BYTES / 16; ++c) {
            u32x4 w = NT ? __builtin_nontemporal_load(q + c) : q[c];
            Word<T>::unpack(w.x, f + (4 * c + 0) * WN);
            Word<T>::unpack(w.y, f + (4 * c + 1) * WN);
            Word<T>::unpack(w.z, f + (4 * c + 2) * WN);
            Word<T>::unpack(w.w, f + (4 * c + 3) * WN);
        }
    } else {
        const u32x2* q = reinterpret_cast<const u32x2*>(p);
#pragma unroll
        for (int c = 0; c < BYTES / 8; ++c) {
            u32x2 w = NT ? __builtin_nontemporal_load(q + c) : q[c];
            Word<T>::unpack(w.x, f + (2 * c + 0) * WN);
            Word<T>::unpack(w.y, f + (2 * c + 1) * WN);
        }
    }
}

template <typename T, int E, bool NT_ = false>
__device__ __forceinline__ void store_elems(T* __restrict__ p, const float* f) {
    constexpr bool NT = NT_ && T2H_NT;
    constexpr int BYTES = E * (int)sizeof(T);
    static_assert(BYTES % 8 == 0, "vector width");
    constexpr int WN = Word<T>::N;
    if constexpr (BYTES % 16 == 0) {
        u32x4* q = reinterpret_cast<u32x4*>(p);
#pragma unroll
        for (int c = 0; c < BYTES / 16; ++c) {
            u32x4 w;
            w.x = Word<T>::pack(f + (4 * c + 0) * WN);
            w.y = Word<T>::pack(f + (4 * c + 1) * WN);
            w.z = Word<T>::pack(f + (4 * c + 2) * WN);
            w.w = Word<T>::pack(f + (4 * c + 3) * WN);
            if (NT) __builtin_nontemporal_store(w, q + c); else q[c] = w;
        }
    } else {
        u32x2* q = reinterpret_cast<u32x2*>(p);
#pragma unroll
        for (int c = 0; c < BYTES / 8; ++c) {
            u32x2 w;
            w.x = Word<T>::pack(f + (2 * c + 0) * WN);
            w.y = Word<T>::pack(f + (2 * c + 1) * WN);
            if (NT) __builtin_nontemporal_store(w, q + c); else q[c] = w;
        }
    }
}

// E contiguous f32 parameters (E multiple of 4 -> 16-byte loads, else scalar).
template <int E>
__device__ __forceinline__ void load_params(const float* __restrict__ p, float* f) {
    if constexpr (E % 4 == 0) {
        const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
        for (int c = 0; c < E / 4; ++c) {
            float4 w = q[c];
            f[4 * c] = w.x; f[4 * c + 1] = w.y; f[4 * c + 2] = w.z; f[4 * c + 3] = w.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < E; ++i) f[i] = p[i];
    }
}

// Scalar element access (fallback kernels).
template <typename T> __device__ __forceinline__ float ld1(const T* p) { return (float)*p; }
template <> __device__ __forceinline__ float ld1<__bf16>(const __bf16* p) {
    return bf16_bits_to_f32(__builtin_bit_cast(uint16_t, *p));
}

// Streams of many non-temporal 16-byte loads run faster on MI355X when a
// small share of the loads (one of a row's three 1 KB pieces in LN, one of a
// gated-residual thread's eight) uses the default cache policy instead:
// LN + modulate 201 -> 188 us, the config-5 chain 1,628 -> 1,601 us. All
// non-temporal, or all cached, is slower. Launches that move less than
// T2H_CACHED_SHARE_MIN bytes keep every load non-temporal: streams that fit
// the 256 MB infinity cache read slower with the share when the cache holds
// other dirty data.
#ifndef T2H_CACHED_SHARE_MIN
#define T2H_CACHED_SHARE_MIN (int64_t(512) << 20)
#endif

// E elements of T (E * sizeof(T) == 16) at element `off` of a wave-uniform
// `row` of `n` elements (n * sizeof(T) <= INT32_MAX: the descriptor's size
// and offset are 32-bit), as f32, with the default (cached) policy: a buffer
// load, a distinct instruction that the compiler does not merge with a
// non-temporal load of the same address under a runtime condition.
template <typename T, int E>
__device__ __forceinline__ void load_elems_cached(const T* row, int64_t off, int64_t n, float* f) {
    if constexpr (E * sizeof(T) != 16) {   // other widths: ordinary cached loads
#pragma unroll
        for (int i = 0; i < E; ++i) f[i] = ld1(row + off + i);
        return;
    }
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(row), 0, (int)(n * (int64_t)sizeof(T)), 0x00020000);
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off * (int64_t)sizeof(T)), 0, 0);
    constexpr int WN = Word<T>::N;
    Word<T>::unpack(w.x, f + 0 * WN);
    Word<T>::unpack(w.y, f + 1 * WN);
    Word<T>::unpack(w.z, f + 2 * WN);
    Word<T>::unpack(w.w, f + 3 * WN);
}

template <typename T> __device__ __forceinline__ void st1(T* p, float v) { *p = (T)v; }
template <> __device__ __forceinline__ void st1<__bf16>(__bf16* p, float v) {
    *p = __builtin_bit_cast(__bf16, (uint16_t)f32_to_bf16_bits(v));
}

// Round-trip through the storage type (what a store + reload yields).
template <typename T> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<_Float16>(float v) { return (float)(_Float16)v; }
template <> __device__ __forceinline__ float round_to<__bf16>(float v) {
    return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// Explicit IEEE single roundings, never contracted into an FMA: the
// bit-exact paths (modulate, gated residual, binop) use these so that
// a*b+c stays two roundings as in the reference. HIP compiles with
// -ffp-contract=fast (and __fmul_rn/__fadd_rn are plain * and +), so the
// operations are emitted without the `contract` flag, which stops the
// backend from fusing them with a neighbouring add/mul after inlining.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

// ---------------------------------------------------------------------------
// DPP reductions (gfx9 DPP controls; all lanes of a row must be active)
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, BANK_MASK, false));
}

// Sum over each DPP row of 16 lanes; every lane of the row gets the same
// value (each step adds a mirrored partner, so all lanes sum identical
// operands in identical pairs).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
}

// Sum over each half DPP row of 8 lanes (lanes 0-7, 8-15 of a row), every
// lane of the half getting the same value.
__device__ __forceinline__ float row8_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    return v;
}

// Sum over the whole wave64; result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// ---------------------------------------------------------------------------
// token row -> parameter row (batch) map
// ---------------------------------------------------------------------------
struct BatchMap {
    const int64_t* offsets;   // [nbatch + 1] or nullptr
    int64_t rows_per_batch;   // > 0: b = r / rows_per_batch
    int32_t nbatch;

    // Largest b in [0, nbatch) with offsets[b] <= r (empty batches skipped,
    // as batch_broadcast_map does).
    __device__ __forceinline__ int32_t batch_of(int64_t r) const {
        if (offsets != nullptr) {
            int32_t lo = 0, hi = nbatch - 1;
            while (lo < hi) {
                const int32_t mid = (lo + hi + 1) >> 1;
                if (offsets[mid] <= r) lo = mid; else hi = mid - 1;
            }
            return lo;
        }
        if (rows_per_batch > 0) return (int32_t)(r / rows_per_batch);
        return 0;
    }
};

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63u); }

// Block barrier that waits only for LDS: lgkmcnt(0) covers this wave's LDS
// stores, and the wave's global loads (vmcnt) stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Linear block index of a launch on grid_1d()'s grid (a second grid
// dimension only past 2^20 blocks; see t2h_internal.h).
__device__ __forceinline__ int64_t block_linear() { return (int64_t)blockIdx.y * gridDim.x + blockIdx.x; }

// Block order over T2H_FRONTS contiguous ranges ("fronts"): physical block
// b runs logical block (b % P) * per + b / P, so P fronts of consecutive
// logical blocks stream at once (front f on XCD f % 8). P = 1: identity.
#ifndef T2H_FRONTS
#define T2H_FRONTS 1
#endif
__device__ __forceinline__ int64_t front_of(int64_t b, int64_t per) {
    if constexpr (T2H_FRONTS == 1) {
        (void)per;
        return b;
    } else {
        return (b % T2H_FRONTS) * per + b / T2H_FRONTS;
    }
}

}  // namespace t2h
