// Device helpers of the in-kernel RoPE: token positions from int voxel coords
// or the dense grid index, and the cos/sin of one rotary slot.
// Reference: sparse/attention/rope.mojo:48-66 (angle = f32(coord) * freq),
// models/sparse_structure_flow.mojo:132-151 (dense 'ij' grid),
// modules/rope.mojo:51-60 (axis-major slots, identity pad slots).
#pragma once
#include "t2h_device.h"

namespace t2h {
namespace {

// Position of token row r along `axis` (f32, exact for |coord| < 2^24).
struct PosSource {
    const int32_t* coords;
    int32_t coord_cols;
    int32_t grid_res;
    int32_t pos_dim;
    __device__ __forceinline__ void get(int64_t r, float* pos) const {
        if (coords != nullptr) {
            const int32_t* cr = coords + r * (int64_t)coord_cols + 1;
#pragma unroll
            for (int ax = 0; ax < T2H_MAX_POS_DIM; ++ax) pos[ax] = ax < pos_dim ? (float)cr[ax] : 0.0f;
        } else {
            const int64_t R = grid_res;
            const int64_t l = r % (R * R * R);
            pos[0] = (float)(l / (R * R));
            pos[1] = (float)((l / R) % R);
            pos[2] = (float)(l % R);
            pos[3] = 0.0f;
        }
    }
};

// Axis of rotary slot p (< head_dim / 2): p / freq_dim for the pos_dim *
// freq_dim rotated slots, -1 (identity) for the pad slots; the same mapping
// as the host's slot table, computed without a load so that a kernel can
// issue its coordinate load at once.
__device__ __forceinline__ int slot_axis(int p, int freq_dim, int pos_dim) {
    return (freq_dim > 0 && p < freq_dim * pos_dim) ? p / freq_dim : -1;
}

__device__ __forceinline__ float pick_axis(const float* pos, int ax) {
    return ax == 0 ? pos[0] : ax == 1 ? pos[1] : ax == 2 ? pos[2] : pos[3];
}

// cos/sin of one slot: angle = pos[axis] * freq rounded to f32, then accurate
// (full-range reduced) cosf/sinf; identity for pad slots (axis < 0).
__device__ __forceinline__ void slot_phase(const float* pos, int ax, float freq, float& c, float& s) {
    if (ax < 0) {
        c = 1.0f;
        s = 0.0f;
    } else {
        const float angle = __fmul_rn(pick_axis(pos, ax), freq);
        sincosf(angle, &s, &c);
    }
}

// One RoPE pair rotation with a fixed rounding sequence (one product and one
// fused multiply-add per output: re*c - im*s = fma(re, c, -fl(im*s))), so
// every kernel that rotates a pair produces the same bits whatever the
// compiler would otherwise contract.
__device__ __forceinline__ void rotate_pair(float& re, float& im, float c, float s) {
    const float a = fmaf(re, c, -mul_rn(im, s));
    const float b = fmaf(re, s, mul_rn(im, c));
    re = a;
    im = b;
}

// Sum of squares of N values in index order, one fused multiply-add each.
template <int N>
__device__ __forceinline__ float sum_sq(const float* x) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) s = fmaf(x[i], x[i], s);
    return s;
}

// Lane layout of one head over LPH lanes (16: a DPP row; 8: half a row):
// lane m holds E = D/LPH elements as NC pieces of VE contiguous elements
// (16 bytes at most), piece j at element j*LPH*VE + m*VE, so every load
// instruction reads one contiguous span across the lanes (f32 with D = 128:
// two 16-byte pieces 256 bytes apart). RoPE pairs (2p, 2p+1) stay inside
// one lane.
template <typename T, int D, int LPH = 16>
struct HeadLanes {
    static_assert(LPH == 16 || LPH == 8, "a head spans a DPP row or half of one");
    static constexpr int E = D / LPH;
    static constexpr int VE = E * (int)sizeof(T) > 16 ? 16 / (int)sizeof(T) : E;
    static constexpr int NC = E / VE;
    static constexpr int P = E / 2;
    __device__ static __forceinline__ int piece(int m, int j) { return j * LPH * VE + m * VE; }
    // element index of the lane's i-th value, and the slot of its pair t
    __device__ static __forceinline__ int elem(int m, int i) { return piece(m, i / VE) + i % VE; }
    __device__ static __forceinline__ int slot(int m, int t) { return elem(m, 2 * t) / 2; }
    __device__ static __forceinline__ void load(const T* head, int m, float* v) {
#pragma unroll
        for (int j = 0; j < NC; ++j) load_elems<T, VE, true>(head + piece(m, j), v + j * VE);
    }
    __device__ static __forceinline__ void store(T* head, int m, const float* v) {
#pragma unroll
        for (int j = 0; j < NC; ++j) store_elems<T, VE, true>(head + piece(m, j), v + j * VE);
    }
    // f32 parameters of the head (bias, gamma) in the lane's order
    __device__ static __forceinline__ void params(const float* head, int m, float* f) {
#pragma unroll
        for (int j = 0; j < NC; ++j) load_params<VE>(head + piece(m, j), f + j * VE);
    }
    // the lane's P (cos, sin) pairs of a phase-table row [D/2][2]
    __device__ static __forceinline__ void phases(const float* row, int m, float* c, float* s) {
        float tmp[E];
#pragma unroll
        for (int j = 0; j < NC; ++j) load_params<VE>(row + piece(m, j), tmp + j * VE);
#pragma unroll
        for (int t = 0; t < P; ++t) { c[t] = tmp[2 * t]; s[t] = tmp[2 * t + 1]; }
    }
};

// v of lane src_lane (ds_bpermute: a lane-indexed read across the wave).
__device__ __forceinline__ float lane_bcast(float v, int src_lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_lane << 2, __builtin_bit_cast(int, v)));
}

}  // namespace
}  // namespace t2h
