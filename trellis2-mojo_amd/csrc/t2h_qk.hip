// Multi-head QK RMSNorm + 3D RoPE (+ qkv bias) on token rows, and the RoPE
// phase-table builder.
//
// Fast path (head_dim 64 or 128, heads <= 16): a block of W waves (8, or 4
// for launches short of rows) handles W consecutive token rows of one tensor (q, k, or the packed
// qkv's v); blocks for the tensors of a row tile are adjacent, so they share
// the tile's coords in cache. Each head is one DPP row of 16 lanes (lane m
// holds E = head_dim/16 elements: one 16-byte piece at m*E, or for f32 with
// head_dim 128 two pieces at m*4 and 64 + m*4, so every load instruction is
// contiguous across the row), so a wave instruction covers 4 heads and the
// per-head sum of squares is a 4-step DPP row sum.
// The interleaved RoPE pairs (2p, 2p+1) are lane-local: lane l computes
// cos/sin of slot l once per row (64 lanes = the 64 slots of head_dim 128)
// from the row's integer voxel coordinate (or the dense grid index), and
// ds_bpermute hands each lane the E/2 slots its pairs need; no phase table is
// read from HBM. The RMS scale is 1/max(sqrt(ss), 1e-12) from v_rsq_f32.
//
// Order inside a wave: slot-coordinate load, then the row loads (all
// unconditional, so they are in flight together), then the block stages the
// tensor's gamma * scale and bias into LDS (no lane reloads a per-head
// parameter from L2) and meets at an LDS-only barrier (lgkmcnt(0) +
// s_barrier). The grid is not persistent: many short blocks stream HBM better on
// MI355X than waves that loop over rows.
//
// Reference: sparse/attention/modules.mojo:37-102 (MultiHeadRMSNorm),
// modules/rope.mojo:17-88, sparse/attention/rope.mojo:20-134 (RoPE),
// gpu/attention.mojo:507-563 (bias_rms_rope_qkv), 596-631 (bias_rms_q).
#include "t2h_device.h"
#include "t2h_internal.h"
#include "t2h_rope.h"

namespace t2h {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

#ifndef T2H_QK_WAVES
#define T2H_QK_WAVES 8
#endif
constexpr int kTileWaves = T2H_QK_WAVES;   // token rows (one per wave) per tile block
constexpr int kSmallTileWaves = 4;         // ... when the launch is short of rows (launch_fast)

template <typename T, int D, int NG, int W, bool EARLY>
__global__ __launch_bounds__(W * 64) void qk_tile_kernel(QkArgs a, RopeSlots tab) {
    // 16-bit rows with D = 64: a head over 8 lanes (16-byte pieces), 8 heads
    // per wave instruction; otherwise 16 lanes, 4 heads
    constexpr int LPH = (sizeof(T) == 2 && D == 64) ? 8 : 16;
    constexpr int HPI = 64 / LPH;
    using L = HeadLanes<T, D, LPH>;
    constexpr int E = L::E;
    constexpr int P = L::P;
    constexpr int VE = L::VE;
    constexpr int HALF = D / 2;
    __shared__ __attribute__((aligned(16))) float gs[NG * HPI * D];   // gamma * scale
    __shared__ __attribute__((aligned(16))) float bs[NG * HPI * D];   // bias (q, k or v)
    const int lane = lane_id();
    const int g = lane / LPH;
    const int m = lane % LPH;
    const int H = a.heads;
    const int HD = H * D;
    const int has_q = a.q_in != nullptr, has_k = a.k_in != nullptr;
    const int has_v = a.v != nullptr && a.bias_v != nullptr;
    const int upr = has_q + has_k + has_v;
    const int64_t b = block_linear();
    int which = (int)(b % upr);   // 0 = q, 1 = k, 2 = v (absent tensors skipped)
    if (!has_q) ++which;
    if (which == 1 && !has_k) ++which;
    const int64_t tile = front_of(b / upr, a.fper);
    if (tile * W >= a.rows) return;   // past the last tile of a 2-D grid (block-uniform)
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r = tile * W + wave;
    const bool live = r < a.rows;
    if (which == 2) {                      // packed qkv: v += bias_v (block-uniform branch)
        // the q/k lane layout over the row's heads, bias_v staged in LDS once
        // per block; every load before the first store (loads and stores
        // share vmcnt on gfx9)
        T* __restrict__ vr = static_cast<T*>(a.v) + (live ? r : a.rows - 1) * a.in_stride;
        float vv[NG][E];
#pragma unroll
        for (int it = 0; it < NG; ++it) {
            const int hh = HPI * it + g;
            L::load(vr + (int64_t)(hh < H ? hh : H - 1) * D, m, vv[it]);
        }
        for (int i = threadIdx.x; i < HD / 4; i += W * 64)
            reinterpret_cast<float4*>(bs)[i] = reinterpret_cast<const float4*>(a.bias_v)[i];
        lds_barrier();
        if (!live) return;
#pragma unroll
        for (int it = 0; it < NG; ++it) {
            const int hh = HPI * it + g;
            if (hh < H) {
                float bv[E];
                L::params(&bs[hh * D], m, bv);
#pragma unroll
                for (int i = 0; i < E; ++i) vv[it][i] = add_rn(vv[it][i], bv[i]);
            }
        }
#pragma unroll
        for (int it = 0; it < NG; ++it) {
            const int hh = HPI * it + g;
            if (hh < H) L::store(vr + (int64_t)hh * D, m, vv[it]);
        }
        return;
    }
    const T* __restrict__ in = static_cast<const T*>(which == 0 ? a.q_in : a.k_in);
    T* __restrict__ out = static_cast<T*>(which == 0 ? a.q_out : a.k_out);
    const float* __restrict__ gamma = which == 0 ? a.gamma_q : a.gamma_k;
    const float* __restrict__ bias = which == 0 ? a.bias_q : a.bias_k;
    const PosSource src{a.coords, a.coord_cols, a.grid_res, a.pos_dim};

    // EARLY (16-bit rows; f32 rows with a bias or in 8-row tiles): the slot's
    // frequency and the block's gamma / bias values are loaded before the
    // row loads, so the phase and the LDS staging wait for them alone and run
    // while the rows are in flight (MI355X, config 5: 414 -> 401 us; the
    // small-T block's packed f32 qkv 116.1 -> 114.4 us per block; config 4's
    // f32 QK 163.8 -> 160.6 us). f32 4-row tiles without a bias keep their
    // parameter loads after the row loads (config 2: 17.7 against 20.8 us
    // early).
    constexpr bool kEarly = EARLY;
    const int my_slot = lane % HALF;
    // 16-bit rows: the slot's axis from its index, so the coordinate load goes
    // out without waiting for a table load (config 5: 402 -> 398 us)
    const int my_axis = kEarly ? slot_axis(my_slot, a.freq_dim, a.pos_dim) : (int)tab.axis[my_slot];
    const float my_freq = kEarly ? tab.freq[my_slot] : 0.0f;
    const bool coord_pos = a.use_rope && a.phases == nullptr && a.coords != nullptr;
    float cpos = 0.0f;
    if (live && coord_pos && my_axis >= 0) cpos = (float)a.coords[r * a.coord_cols + 1 + my_axis];

    // gamma * scale and the bias, staged in LDS once per block. A thread
    // holds at most two float4s of each in named registers: an array indexed
    // by a loop counter is placed in LDS (or scratch) by the compiler before
    // the loop is unrolled, and its store would wait for the parameter load
    // ahead of the row loads
    constexpr int KP = (NG * HPI * D / 4 + W * 64 - 1) / (W * 64);   // parameter float4s per thread
    static_assert(KP <= 2, "parameter float4s per thread");
    const bool stage = gamma != nullptr || bias != nullptr;   // block-uniform
    const int pi0 = threadIdx.x, pi1 = threadIdx.x + W * 64;
    float4 gl0 = make_float4(0.f, 0.f, 0.f, 0.f), gl1 = gl0, bl0 = gl0, bl1 = gl0;
    if constexpr (kEarly) {
        if (gamma != nullptr && pi0 < HD / 4) gl0 = reinterpret_cast<const float4*>(gamma)[pi0];
        if (bias != nullptr && pi0 < HD / 4) bl0 = reinterpret_cast<const float4*>(bias)[pi0];
        if (KP > 1 && gamma != nullptr && pi1 < HD / 4) gl1 = reinterpret_cast<const float4*>(gamma)[pi1];
        if (KP > 1 && bias != nullptr && pi1 < HD / 4) bl1 = reinterpret_cast<const float4*>(bias)[pi1];
    }
    const int64_t rl = live ? r : a.rows - 1;   // dead waves load a valid row, store nothing
    float v[NG][E];
#pragma unroll
    for (int it = 0; it < NG; ++it) {
        const int hh = HPI * it + g;
        const int hl = hh < H ? hh : H - 1;
        L::load(in + rl * a.in_stride + (int64_t)hl * D, m, v[it]);
    }
    if constexpr (kEarly) {
        const float sc = a.rms_scale;
        if (gamma != nullptr && pi0 < HD / 4)
            reinterpret_cast<float4*>(gs)[pi0] = make_float4(gl0.x * sc, gl0.y * sc, gl0.z * sc, gl0.w * sc);
        if (bias != nullptr && pi0 < HD / 4) reinterpret_cast<float4*>(bs)[pi0] = bl0;
        if (KP > 1 && gamma != nullptr && pi1 < HD / 4)
            reinterpret_cast<float4*>(gs)[pi1] = make_float4(gl1.x * sc, gl1.y * sc, gl1.z * sc, gl1.w * sc);
        if (KP > 1 && bias != nullptr && pi1 < HD / 4) reinterpret_cast<float4*>(bs)[pi1] = bl1;
    } else {
        if (gamma != nullptr) {
            for (int i = threadIdx.x; i < HD; i += W * 64) gs[i] = gamma[i] * a.rms_scale;
        }
        if (bias != nullptr) {
            for (int i = threadIdx.x; i < HD / 4; i += W * 64)
                reinterpret_cast<float4*>(bs)[i] = reinterpret_cast<const float4*>(bias)[i];
        }
    }

    float pc[P], ps[P];
    if (a.use_rope) {
        if (a.phases != nullptr) {
            const int64_t l = live ? r % a.phase_rows : 0;
            L::phases(a.phases + l * HALF * 2, m, pc, ps);
        } else {
            float pos[T2H_MAX_POS_DIM] = {cpos, cpos, cpos, cpos};
            if (!coord_pos) src.get(live ? r : 0, pos);
            float c, s;
            slot_phase(pos, my_axis, kEarly ? my_freq : tab.freq[my_slot], c, s);
#pragma unroll
            for (int t = 0; t < P; ++t) {
                pc[t] = lane_bcast(c, L::slot(m, t));
                ps[t] = lane_bcast(s, L::slot(m, t));
            }
        }
    }

    if (stage) lds_barrier();
    if (!live) return;

#pragma unroll
    for (int it = 0; it < NG; ++it) {
        const int hh = HPI * it + g;
        const bool valid = hh < H;
        if (bias != nullptr && valid) {
            float bv[E];
            L::params(&bs[hh * D], m, bv);
#pragma unroll
            for (int i = 0; i < E; ++i) v[it][i] = add_rn(v[it][i], bv[i]);
        }
        if (gamma != nullptr) {
            float ss = sum_sq<E>(v[it]);
            if constexpr (LPH == 16) ss = row16_sum(ss);
            else ss = row8_sum(ss);
            const float rn = ss < 1e-24f ? 1e12f : __builtin_amdgcn_rsqf(ss);
            float gv[E];
#pragma unroll
            for (int j = 0; j < L::NC; ++j) {
                const float4* gp = reinterpret_cast<const float4*>(&gs[(valid ? hh : 0) * D + L::piece(m, j)]);
#pragma unroll
                for (int c4 = 0; c4 < VE / 4; ++c4) {
                    const float4 w = gp[c4];
                    float* d = &gv[j * VE + 4 * c4];
                    d[0] = w.x; d[1] = w.y; d[2] = w.z; d[3] = w.w;
                }
            }
#pragma unroll
            for (int i = 0; i < E; ++i) v[it][i] = (v[it][i] * rn) * gv[i];
        }
        if (a.use_rope) {
#pragma unroll
            for (int t = 0; t < P; ++t) rotate_pair(v[it][2 * t], v[it][2 * t + 1], pc[t], ps[t]);
        }
        if (valid) L::store(out + r * a.out_stride + (int64_t)hh * D, m, v[it]);
    }
}

// Any even head_dim / any head count: one wave per (row, head); lanes stride
// over the pairs of the head.
template <typename T>
__global__ __launch_bounds__(kBlock) void qk_rows_generic(QkArgs a, RopeSlots tab) {
    const int lane = lane_id();
    const int D = a.head_dim, half = D / 2, H = a.heads;
    const T* __restrict__ qi = static_cast<const T*>(a.q_in);
    const T* __restrict__ ki = static_cast<const T*>(a.k_in);
    T* __restrict__ qo = static_cast<T*>(a.q_out);
    T* __restrict__ ko = static_cast<T*>(a.k_out);
    const PosSource src{a.coords, a.coord_cols, a.grid_res, a.pos_dim};
    const int64_t units = a.rows * H;
    const int64_t nwaves = (int64_t)gridDim.x * kWaves;
    for (int64_t u = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); u < units; u += nwaves) {
        const int64_t r = u / H;
        const int hh = (int)(u % H);
        float pos[T2H_MAX_POS_DIM];
        if (a.use_rope && a.phases == nullptr) src.get(r, pos);
        for (int which = 0; which < 2; ++which) {
            const T* in = which == 0 ? qi : ki;
            if (in == nullptr) continue;
            T* out = which == 0 ? qo : ko;
            const float* bias = which == 0 ? a.bias_q : a.bias_k;
            const float* gm = which == 0 ? a.gamma_q : a.gamma_k;
            const int64_t ib = r * a.in_stride + (int64_t)hh * D;
            const int64_t ob = r * a.out_stride + (int64_t)hh * D;
            float ss = 0.0f;
            for (int p = lane; p < half; p += 64) {
                float re = ld1(in + ib + 2 * p), im = ld1(in + ib + 2 * p + 1);
                if (bias) { re = add_rn(re, bias[hh * D + 2 * p]); im = add_rn(im, bias[hh * D + 2 * p + 1]); }
                ss += re * re + im * im;
            }
            float rn = 1.0f;
            if (gm != nullptr) {
                ss = wave_sum(ss);
                float nrm = sqrtf(ss);
                if (nrm < 1e-12f) nrm = 1e-12f;
                rn = 1.0f / nrm;
            }
            for (int p = lane; p < half; p += 64) {
                float re = ld1(in + ib + 2 * p), im = ld1(in + ib + 2 * p + 1);
                if (bias) { re = add_rn(re, bias[hh * D + 2 * p]); im = add_rn(im, bias[hh * D + 2 * p + 1]); }
                if (gm != nullptr) {
                    re = re * rn * gm[hh * D + 2 * p] * a.rms_scale;
                    im = im * rn * gm[hh * D + 2 * p + 1] * a.rms_scale;
                }
                if (a.use_rope) {
                    float c, s;
                    if (a.phases != nullptr) {
                        const int64_t l = r % a.phase_rows;
                        c = a.phases[(l * half + p) * 2];
                        s = a.phases[(l * half + p) * 2 + 1];
                    } else {
                        slot_phase(pos, tab.axis[p], tab.freq[p], c, s);
                    }
                    const float nre = re * c - im * s;
                    const float nim = re * s + im * c;
                    re = nre;
                    im = nim;
                }
                st1(out + ob + 2 * p, re);
                st1(out + ob + 2 * p + 1, im);
            }
        }
        if (a.v != nullptr && a.bias_v != nullptr) {
            T* vr = static_cast<T*>(a.v) + r * a.in_stride + (int64_t)hh * D;
            for (int e = lane; e < D; e += 64) st1(vr + e, add_rn(ld1(vr + e), a.bias_v[hh * D + e]));
        }
    }
}

// Phase table [rows, D/2, 2]: one thread per (row, slot).
__global__ __launch_bounds__(kBlock) void phases_kernel(PhaseArgs a, RopeSlots tab) {
    const int half = a.head_dim / 2;
    const int64_t total = a.rows * half;
    const PosSource src{a.coords, a.coord_cols, a.grid_res, a.pos_dim};
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
        const int64_t r = i / half;
        const int p = (int)(i % half);
        float pos[T2H_MAX_POS_DIM];
        if (a.positions != nullptr) {
#pragma unroll
            for (int ax = 0; ax < T2H_MAX_POS_DIM; ++ax)
                pos[ax] = ax < a.pos_dim ? a.positions[r * a.pos_dim + ax] : 0.0f;
        } else {
            src.get(r, pos);
        }
        float c, s;
        slot_phase(pos, tab.axis[p], tab.freq[p], c, s);
        reinterpret_cast<float2*>(a.out)[i] = make_float2(c, s);
    }
}

template <typename K>
int resident_blocks(K kernel) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, kBlock, 0) != hipSuccess || nb <= 0) nb = 2;
    return nb * device_cu_count();
}

// Rows per tile block: 8 waves, or 4 when 8-row tiles would give fewer than
// 8 blocks per CU (e.g. the dense 16^3 grid's 4096 rows: 3.7 % faster in
// back-to-back launches; at 200k rows 4-row tiles are 9 % slower).
template <typename T, int D, int NG>
hipError_t launch_fast(QkArgs a, const RopeSlots& tab, hipStream_t s) {
    const int upr = (a.q_in != nullptr) + (a.k_in != nullptr) + (a.v != nullptr && a.bias_v != nullptr);
    const bool small = (a.rows + kTileWaves - 1) / kTileWaves * upr < 8LL * device_cu_count();
    const int w = small ? kSmallTileWaves : kTileWaves;
    const int64_t tiles = (a.rows + w - 1) / w;
    a.fper = front_per(tiles);
    const dim3 grid = grid_1d(front_grid(tiles) * upr);
    if constexpr (sizeof(T) == 2) {
        if (small) hipLaunchKernelGGL((qk_tile_kernel<T, D, NG, kSmallTileWaves, true>), grid, dim3(kSmallTileWaves * 64), 0, s, a, tab);
        else hipLaunchKernelGGL((qk_tile_kernel<T, D, NG, kTileWaves, true>), grid, dim3(kTileWaves * 64), 0, s, a, tab);
    } else if (a.bias_q != nullptr || a.bias_k != nullptr || !small) {
        if (small) hipLaunchKernelGGL((qk_tile_kernel<T, D, NG, kSmallTileWaves, true>), grid, dim3(kSmallTileWaves * 64), 0, s, a, tab);
        else hipLaunchKernelGGL((qk_tile_kernel<T, D, NG, kTileWaves, true>), grid, dim3(kTileWaves * 64), 0, s, a, tab);
    } else {
        if (small) hipLaunchKernelGGL((qk_tile_kernel<T, D, NG, kSmallTileWaves, false>), grid, dim3(kSmallTileWaves * 64), 0, s, a, tab);
        else hipLaunchKernelGGL((qk_tile_kernel<T, D, NG, kTileWaves, false>), grid, dim3(kTileWaves * 64), 0, s, a, tab);
    }
    return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_d(const QkArgs& a, const RopeSlots& tab, hipStream_t s) {
    if constexpr (sizeof(T) == 2 && D == 64) {   // 8 heads per group (8 lanes per head)
        if (a.heads <= 8) return launch_fast<T, D, 1>(a, tab, s);
        return launch_fast<T, D, 2>(a, tab, s);
    } else {
        switch ((a.heads + 3) / 4) {
            case 1: return launch_fast<T, D, 1>(a, tab, s);
            case 2: return launch_fast<T, D, 2>(a, tab, s);
            case 3: return launch_fast<T, D, 3>(a, tab, s);
            default: return launch_fast<T, D, 4>(a, tab, s);
        }
    }
}

inline bool aligned_to(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

template <typename T>
hipError_t launch_typed(const QkArgs& a, const RopeSlots& tab, hipStream_t s) {
    // vector loads of min(16, E * sizeof(T)) bytes per lane need that
    // alignment (E = head_dim / lanes per head: 8 lanes for 16-bit D = 64)
    const int lph = sizeof(T) == 2 && a.head_dim == 64 ? 8 : 16;
    const int E = a.head_dim / lph;
    const int chunk = E * (int)sizeof(T) < 16 ? E * (int)sizeof(T) : 16;
    const int64_t ealign = chunk / (int64_t)sizeof(T);
    const bool aligned = (a.in_stride % ealign == 0) && (a.out_stride % ealign == 0) &&
                         aligned_to(a.q_in, chunk) && aligned_to(a.k_in, chunk) &&
                         aligned_to(a.q_out, chunk) && aligned_to(a.k_out, chunk) &&
                         aligned_to(a.v, chunk) && aligned_to(a.bias_q, 16) && aligned_to(a.bias_k, 16) &&
                         aligned_to(a.bias_v, 16) && aligned_to(a.gamma_q, 16) &&
                         aligned_to(a.gamma_k, 16) && aligned_to(a.phases, 16);
    if (a.heads <= 16 && aligned) {
        if (a.head_dim == 128) return launch_d<T, 128>(a, tab, s);
        if (a.head_dim == 64) return launch_d<T, 64>(a, tab, s);
    }
    auto k = qk_rows_generic<T>;
    static const int cap = resident_blocks(k);
    const int64_t need = (a.rows * a.heads + kWaves - 1) / kWaves;
    const int grid = (int)(need < cap ? need : cap);
    hipLaunchKernelGGL(k, dim3(grid), dim3(kBlock), 0, s, a, tab);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_qk(const QkArgs& a, const RopeSlots& tab, hipStream_t s) {
    switch (a.dtype) {
        case T2H_F32: return launch_typed<float>(a, tab, s);
        case T2H_F16: return launch_typed<_Float16>(a, tab, s);
        default: return launch_typed<__bf16>(a, tab, s);
    }
}

hipError_t launch_phases(const PhaseArgs& a, const RopeSlots& tab, hipStream_t s) {
    const int64_t total = a.rows * (a.head_dim / 2);
    int64_t grid = (total + kBlock - 1) / kBlock;
    const int64_t cap = 64LL * device_cu_count();
    if (grid > cap) grid = cap;
    hipLaunchKernelGGL(phases_kernel, dim3((unsigned)grid), dim3(kBlock), 0, s, a, tab);
    return hipGetLastError();
}

}  // namespace t2h
