// Self-attention epilogue fused with the head-major packing of the attention
// operands: one pass over the qkv GEMM output instead of an in-place epilogue
// pass followed by two packing passes.
//
//   q, k, v [rows, H, D] (rows in_stride apart, e.g. views of a packed qkv
//   [rows, 3, H, D]) --(+bias, RMS q/k, RoPE q/k)-->
//   qh [H, mp, D] = q * 1/sqrt(D); k_out [H, D, lp] (transposed) or
//   [H, lp, D]; vh [H, lp, D]; pad rows rows..mp-1 / rows..lp-1 are zero.
//
// Two kernels:
// - pack_rows_kernel (row-major outputs: qh, k as [H, lp, D], vh; <= 16
//   heads): one wave per token row reads the tensor's whole row with
//   contiguous 16-byte lanes; each 16-lane DPP row holds one head (lane m:
//   elements [m*E, m*E+E), E = D/16), so the per-head sum of squares is a
//   4-step DPP row sum and one sincos per lane per row serves every head.
//   Each head's rows land as contiguous runs of the head-major output; for
//   16-bit rows of head_dim 128 the block stages its rows in LDS and writes
//   each head's run of 8 rows (2 KB) with whole 1 KB store instructions.
// - pack_tile_kernel (the reference's transposed k [H, D, lp], and row-major
//   outputs beyond 16 heads): a block of 4 waves takes 64 token rows of one
//   tensor and loops over a group of heads; a wave instruction covers 4 rows
//   of one head, the rows' cos/sin stay in registers across the heads. The
//   transposed k goes through LDS (f32: 64 x (D+1), odd row pitch,
//   conflict-free column reads; 16-bit: the output bits in two 64 x (D+2)
//   buffers, one per alternate head, so one barrier per head) and leaves as
//   16-byte vectors along the token axis.
// On MI355X the row-major k ([H, lp, D]) is the faster layout: its rows are
// what an MFMA attention kernel reads as the K operand.
//
// Reference: gpu/attention.mojo:507-563 (bias_rms_rope_qkv), 566-594
// (pack_q_z), 634-662 (pack_kv_z), sequence 987-1013; cross chain q:
// 596-631 (bias_rms_q) + pack_q_z with stride H*D (sequence 1223-1234).
#include "t2h_device.h"
#include "t2h_internal.h"
#include "t2h_rope.h"

namespace t2h {
namespace {

#ifndef T2H_PACK_ROWS
#define T2H_PACK_ROWS 64
#endif
constexpr int kPackRows = T2H_PACK_ROWS;   // token rows per tile block
#ifndef T2H_PACK_WAVES
#define T2H_PACK_WAVES 4
#endif
constexpr int kPackBlock = 64 * T2H_PACK_WAVES;
constexpr int kPackRowsPerIter = 4 * T2H_PACK_WAVES;         // a wave instruction covers 4 rows
constexpr int kPackIters = kPackRows / kPackRowsPerIter;    // row groups of 4 per wave
static_assert(kPackIters * kPackRowsPerIter == kPackRows, "tile rows");

// One lane's E elements of one head row, held as the loaded 32-bit words so
// that a prefetch stays in flight until the words are unpacked.
template <typename T, int D>
struct RawRow {
    using L = HeadLanes<T, D>;
    static constexpr int WP = L::VE * (int)sizeof(T) / 4;   // words per piece
    static_assert(WP == 2 || WP == 4, "piece width");
    uint32_t w[L::NC * WP];
    __device__ __forceinline__ void load(const T* head, int m) {
#pragma unroll
        for (int j = 0; j < L::NC; ++j) {
            const T* p = head + L::piece(m, j);
            if constexpr (WP == 4) {
                const u32x4 q = T2H_NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p))
                                       : *reinterpret_cast<const u32x4*>(p);
                w[j * 4 + 0] = q.x;
                w[j * 4 + 1] = q.y;
                w[j * 4 + 2] = q.z;
                w[j * 4 + 3] = q.w;
            } else {
                const u32x2 q = T2H_NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p))
                                       : *reinterpret_cast<const u32x2*>(p);
                w[j * 2 + 0] = q.x;
                w[j * 2 + 1] = q.y;
            }
        }
    }
    __device__ __forceinline__ void unpack(float* v) const {
#pragma unroll
        for (int k = 0; k < L::NC * WP; ++k) Word<T>::unpack(w[k], v + k * Word<T>::N);
    }
};

// The 1-D grid covers row tiles x tensors x head groups, head groups varying
// fastest. which[] maps the tensor index to the tensor a block packs
// (0 = q, 1 = k, 2 = v); a block loops over the `hpb` heads of its group, so
// the RoPE cos/sin of its rows, computed once into registers, serve every
// head of the group.
struct PackOrder {
    int32_t n;        // tensors in this launch
    int32_t groups;   // head groups = heads / hpb
    int32_t hpb;      // heads per block
    int8_t which[3];
};

template <typename T, int D, bool KT>
__global__ __launch_bounds__(kPackBlock) void pack_tile_kernel(PackArgs a, RopeSlots tab, PackOrder order) {
    using L = HeadLanes<T, D>;
    constexpr int E = L::E;
    constexpr int P = L::P;
    // The transposed tile: f32 rows, one buffer (two barriers per head); for
    // 16-bit storage the output bit patterns in two buffers, so a head's tile
    // is written while the previous head's is read (one barrier per head).
    constexpr bool kTwo = KT && sizeof(T) == 2;
    __shared__ float tile[KT && !kTwo ? kPackRows : 1][KT && !kTwo ? D + 1 : 1];
    __shared__ uint16_t tile2[kTwo ? 2 : 1][kTwo ? kPackRows : 1][kTwo ? D + 2 : 1];
    const int lane = lane_id();
    const int g = lane >> 4;
    const int m = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t b = block_linear();
    const int hg = (int)(b % order.groups);
    const int which = order.which[(b / order.groups) % order.n];
    const int64_t t0 = (b / ((int64_t)order.groups * order.n)) * kPackRows;
    const int64_t extent = which == 0 ? a.mp : a.lp;
    if (t0 >= extent) return;

    const T* __restrict__ in = static_cast<const T*>(which == 0 ? a.q : which == 1 ? a.k : a.v);
    T* __restrict__ out = static_cast<T*>(which == 0 ? a.qh : which == 1 ? a.k_out : a.vh);
    const float* __restrict__ bias = which == 0 ? a.bias_q : which == 1 ? a.bias_k : a.bias_v;
    const float* __restrict__ gamma = which == 0 ? a.gamma_q : which == 1 ? a.gamma_k : nullptr;
    // with no token rows every output is a pad: no phase (coords) or row read
    const bool rope = a.use_rope && which < 2 && a.rows > 0;

    // this lane's token rows (clamped for the loads; rows >= a.rows are pads)
    int64_t rl[kPackIters];
#pragma unroll
    for (int it = 0; it < kPackIters; ++it) {
        const int64_t t = t0 + it * kPackRowsPerIter + wave * 4 + g;
        rl[it] = t < a.rows ? t : (a.rows > 0 ? a.rows - 1 : 0);
    }

    // cos/sin of this lane's P slots for each of its rows, shared by all heads
    float pc[kPackIters][P], ps[kPackIters][P];
    if (rope) {
        if (a.phases != nullptr) {
#pragma unroll
            for (int it = 0; it < kPackIters; ++it) {
                const int64_t l = rl[it] % a.phase_rows;
                L::phases(a.phases + l * D, m, pc[it], ps[it]);
            }
        } else {
            const PosSource src{a.coords, a.coord_cols, a.grid_res, a.pos_dim};
            int ax[P];
            float fr[P];
#pragma unroll
            for (int j = 0; j < P; ++j) {
                ax[j] = tab.axis[L::slot(m, j)];
                fr[j] = tab.freq[L::slot(m, j)];
            }
#pragma unroll
            for (int it = 0; it < kPackIters; ++it) {
                float pos[T2H_MAX_POS_DIM];
                src.get(rl[it], pos);
#pragma unroll
                for (int j = 0; j < P; ++j) slot_phase(pos, ax[j], fr[j], pc[it][j], ps[it][j]);
            }
        }
    }

    // The transposed path fetches head z + 1 (rows and the head's bias and
    // gamma) before it stores head z, so a block's loads overlap its own
    // stores and no parameter load waits for them (loads and stores share
    // vmcnt on gfx9).
    RawRow<T, D> raw[kPackIters];
    float bv[E], gv[E];
    auto fetch = [&](int z) {
        if (a.rows > 0) {
#pragma unroll
            for (int it = 0; it < kPackIters; ++it) raw[it].load(in + rl[it] * a.in_stride + (int64_t)z * D, m);
        }
        if (bias != nullptr) L::params(bias + z * D, m, bv);
        if (gamma != nullptr) L::params(gamma + z * D, m, gv);
    };
    if constexpr (KT) fetch(hg * order.hpb);
    for (int zi = 0; zi < order.hpb; ++zi) {
        const int z = hg * order.hpb + zi;
        if constexpr (!KT) fetch(z);
        float v[kPackIters][E];
        if (a.rows > 0) {
#pragma unroll
            for (int it = 0; it < kPackIters; ++it) raw[it].unpack(v[it]);
        } else {
#pragma unroll
            for (int it = 0; it < kPackIters; ++it)
#pragma unroll
                for (int i = 0; i < E; ++i) v[it][i] = 0.0f;
        }
        float gsc[E];
        if (gamma != nullptr) {
#pragma unroll
            for (int i = 0; i < E; ++i) gsc[i] = gv[i] * a.rms_scale;
        }
#pragma unroll
        for (int it = 0; it < kPackIters; ++it) {
            const int64_t t = t0 + it * kPackRowsPerIter + wave * 4 + g;
            float* x = v[it];
            if (bias != nullptr) {
#pragma unroll
                for (int i = 0; i < E; ++i) x[i] = add_rn(x[i], bv[i]);
            }
            if (gamma != nullptr) {
                const float ss = row16_sum(sum_sq<E>(x));
                const float rn = ss < 1e-24f ? 1e12f : __builtin_amdgcn_rsqf(ss);
#pragma unroll
                for (int i = 0; i < E; ++i) x[i] = (x[i] * rn) * gsc[i];
            }
            if (rope) {
#pragma unroll
                for (int j = 0; j < P; ++j) rotate_pair(x[2 * j], x[2 * j + 1], pc[it][j], ps[it][j]);
            }
            if (which == 0) {
#pragma unroll
                for (int i = 0; i < E; ++i) x[i] = mul_rn(x[i], a.q_scale);
            }
            if (t >= a.rows) {
#pragma unroll
                for (int i = 0; i < E; ++i) x[i] = 0.0f;
            }
            if constexpr (kTwo) {
                // elements 2i, 2i+1 of a lane are adjacent (pieces of >= 2 elements)
                const int tl = it * kPackRowsPerIter + wave * 4 + g;
#pragma unroll
                for (int i = 0; i < E; i += 2) {
                    const uint32_t w = Word<T>::pack(x + i);
                    tile2[zi & 1][tl][L::elem(m, i)] = (uint16_t)w;
                    tile2[zi & 1][tl][L::elem(m, i) + 1] = (uint16_t)(w >> 16);
                }
            } else if constexpr (KT) {
                const int tl = it * kPackRowsPerIter + wave * 4 + g;
#pragma unroll
                for (int i = 0; i < E; ++i) tile[tl][L::elem(m, i)] = round_to<T>(x[i]);
            } else if (t < extent) {
                L::store(out + ((int64_t)z * extent + t) * D, m, x);
            }
        }
        if constexpr (kTwo) {
            // this head's tile is whole, and every read of the tile written
            // two heads ago (the other buffer's previous contents) is done
            __syncthreads();
            if (zi + 1 < order.hpb) fetch(z + 1);
            constexpr int VE = kPack<T>;
            constexpr int VPR = kPackRows / VE;
            for (int vi = threadIdx.x; vi < D * VPR; vi += kPackBlock) {
                const int e = vi / VPR;
                const int tq = (vi % VPR) * VE;
                if (t0 + tq >= extent) continue;
                uint16_t w[VE];
#pragma unroll
                for (int i = 0; i < VE; ++i) w[i] = tile2[zi & 1][tq + i][e];
                u32x4 o;
                __builtin_memcpy(&o, w, 16);
                u32x4* dst = reinterpret_cast<u32x4*>(out + ((int64_t)z * D + e) * a.lp + t0 + tq);
                if (T2H_NT) __builtin_nontemporal_store(o, dst); else *dst = o;
            }
        } else if constexpr (KT) {
            __syncthreads();
            if (zi + 1 < order.hpb) fetch(z + 1);
            constexpr int VE = kPack<T>;            // elements per 16-byte vector
            constexpr int VPR = kPackRows / VE;     // vectors per output row (one e)
            for (int vi = threadIdx.x; vi < D * VPR; vi += kPackBlock) {
                const int e = vi / VPR;
                const int tq = (vi % VPR) * VE;
                if (t0 + tq >= extent) continue;
                float w[VE];
#pragma unroll
                for (int i = 0; i < VE; ++i) w[i] = tile[tq + i][e];
                store_elems<T, VE, true>(out + ((int64_t)z * D + e) * a.lp + t0 + tq, w);
            }
            __syncthreads();
        }
    }
}

// Row-major outputs (qh, k as [H, lp, D], vh) for up to 16 heads: one wave
// per token row, reading the tensor's whole row (all heads) with contiguous
// 16-byte lanes, as the QK kernel does. Lane l computes cos/sin of slot l of
// its row once and ds_bpermute hands each lane the E/2 slots it needs, so the
// rotation costs one sincos per lane per row for every head. gamma * scale is
// staged in LDS behind an LDS-only barrier (lgkmcnt(0) + s_barrier) that
// leaves the row loads in flight. Blocks of the q, k and v of a row tile are
// adjacent, so the qkv rows are read whole.
constexpr int kRowWaves = 8;
constexpr int kRowBlock = kRowWaves * 64;

template <typename T, int D, int NG>
__global__ __launch_bounds__(kRowBlock) void pack_rows_kernel(PackArgs a, RopeSlots tab, PackOrder order) {
    using L = HeadLanes<T, D>;
    constexpr int E = L::E;
    constexpr int P = L::P;
    constexpr int VE = L::VE;
    constexpr int HALF = D / 2;
    constexpr int KP = (NG * 4 * D + kRowBlock - 1) / kRowBlock;   // parameter values per thread
    __shared__ __attribute__((aligned(16))) float gs[NG * 4 * D];   // gamma * scale
    __shared__ __attribute__((aligned(16))) float bs[NG * 4 * D];   // bias
    // 16-bit: the block's rows staged per head, then written as whole
    // per-head runs of the tile's rows (kRowWaves * D * 2 bytes each)
    constexpr bool kStage = sizeof(T) == 2 && VE * (int)sizeof(T) == 16 && L::NC == 1;
    __shared__ __attribute__((aligned(16))) T ost[kStage ? kRowWaves : 1][kStage ? NG * 4 * D : 1];
    const int lane = lane_id();
    const int g = lane >> 4;
    const int m = lane & 15;
    const int H = a.heads;
    const int64_t b = block_linear();
    const int which = order.which[b % order.n];
    const int64_t tile = b / order.n;
    const int64_t extent = which == 0 ? a.mp : a.lp;
    if (tile * kRowWaves >= extent) return;   // block-uniform
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r = tile * kRowWaves + wave;
    const bool live = r < a.rows;

    const T* __restrict__ in = static_cast<const T*>(which == 0 ? a.q : which == 1 ? a.k : a.v);
    T* __restrict__ out = static_cast<T*>(which == 0 ? a.qh : which == 1 ? a.k_out : a.vh);
    const float* __restrict__ bias = which == 0 ? a.bias_q : which == 1 ? a.bias_k : a.bias_v;
    const float* __restrict__ gamma = which == 0 ? a.gamma_q : which == 1 ? a.gamma_k : nullptr;
    const bool rope = a.use_rope && which < 2 && a.rows > 0;   // no rows: all pads

    // 16-bit rows: the slot's frequency and the tensor's gamma and bias
    // values are loaded before the row loads, so the phase and the LDS
    // staging wait for them alone (as in qk_tile_kernel); f32 stages its
    // parameters after the row loads.
    constexpr bool kEarly = sizeof(T) == 2;
    const int my_slot = lane % HALF;
    const int my_axis = tab.axis[my_slot];
    const float my_freq = kEarly ? tab.freq[my_slot] : 0.0f;
    const bool coord_pos = rope && a.phases == nullptr && a.coords != nullptr;
    float cpos = 0.0f;
    if (live && coord_pos && my_axis >= 0) cpos = (float)a.coords[r * a.coord_cols + 1 + my_axis];

    // the tensor's gamma and bias rows, staged in LDS once per block
    const bool stage = gamma != nullptr || bias != nullptr;   // block-uniform
    float gl[KP], bl[KP];
    if constexpr (kEarly) {
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            const int i = threadIdx.x + k * kRowBlock;
            if (gamma != nullptr && i < H * D) gl[k] = gamma[i];
            if (bias != nullptr && i < H * D) bl[k] = bias[i];
        }
    }
    const int64_t rl = live ? r : (a.rows > 0 ? a.rows - 1 : 0);
    float v[NG][E];
    if (a.rows > 0) {
#pragma unroll
        for (int it = 0; it < NG; ++it) {
            const int hh = 4 * it + g;
            const int hl = hh < H ? hh : H - 1;
            L::load(in + rl * a.in_stride + (int64_t)hl * D, m, v[it]);
        }
    } else {
#pragma unroll
        for (int it = 0; it < NG; ++it)
#pragma unroll
            for (int i = 0; i < E; ++i) v[it][i] = 0.0f;
    }
    if constexpr (kEarly) {
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            const int i = threadIdx.x + k * kRowBlock;
            if (gamma != nullptr && i < H * D) gs[i] = gl[k] * a.rms_scale;
            if (bias != nullptr && i < H * D) bs[i] = bl[k];
        }
    } else {
        for (int i = threadIdx.x; i < H * D; i += kRowBlock) {
            if (gamma != nullptr) gs[i] = gamma[i] * a.rms_scale;
            if (bias != nullptr) bs[i] = bias[i];
        }
    }
    float pc[P], ps[P];
    if (rope) {
        if (a.phases != nullptr) {
            const int64_t l = rl % a.phase_rows;
            L::phases(a.phases + l * HALF * 2, m, pc, ps);
        } else {
            float pos[T2H_MAX_POS_DIM] = {cpos, cpos, cpos, cpos};
            if (!coord_pos) {
                const PosSource src{a.coords, a.coord_cols, a.grid_res, a.pos_dim};
                src.get(rl, pos);
            }
            float c, sn;
            slot_phase(pos, my_axis, kEarly ? my_freq : tab.freq[my_slot], c, sn);
#pragma unroll
            for (int t = 0; t < P; ++t) {
                pc[t] = lane_bcast(c, L::slot(m, t));
                ps[t] = lane_bcast(sn, L::slot(m, t));
            }
        }
    }
    if (stage) lds_barrier();
    if (!kStage && r >= extent) return;

#pragma unroll
    for (int it = 0; it < NG; ++it) {
        const int hh = 4 * it + g;
        if (hh >= H) continue;   // uniform over the 16-lane row
        float* x = v[it];
        if (bias != nullptr) {
            float bv[E];
            L::params(&bs[hh * D], m, bv);
#pragma unroll
            for (int i = 0; i < E; ++i) x[i] = add_rn(x[i], bv[i]);
        }
        if (gamma != nullptr) {
            const float ss = row16_sum(sum_sq<E>(x));
            const float rn = ss < 1e-24f ? 1e12f : __builtin_amdgcn_rsqf(ss);
#pragma unroll
            for (int j = 0; j < L::NC; ++j) {
                const float4* gp = reinterpret_cast<const float4*>(&gs[hh * D + L::piece(m, j)]);
#pragma unroll
                for (int c4 = 0; c4 < VE / 4; ++c4) {
                    const float4 w = gp[c4];
                    float* d = &x[j * VE + 4 * c4];
                    d[0] = (d[0] * rn) * w.x;
                    d[1] = (d[1] * rn) * w.y;
                    d[2] = (d[2] * rn) * w.z;
                    d[3] = (d[3] * rn) * w.w;
                }
            }
        }
        if (rope) {
#pragma unroll
            for (int t = 0; t < P; ++t) rotate_pair(x[2 * t], x[2 * t + 1], pc[t], ps[t]);
        }
        if (which == 0) {
#pragma unroll
            for (int i = 0; i < E; ++i) x[i] = mul_rn(x[i], a.q_scale);
        }
        if (!live) {
#pragma unroll
            for (int i = 0; i < E; ++i) x[i] = 0.0f;
        }
        if constexpr (kStage) {
            uint32_t w[VE / 2];
#pragma unroll
            for (int i = 0; i < VE / 2; ++i) w[i] = Word<T>::pack(x + 2 * i);
            u32x4 o;
            __builtin_memcpy(&o, w, 16);
            *reinterpret_cast<u32x4*>(&ost[wave][hh * D + m * VE]) = o;
        } else {
            L::store(out + ((int64_t)hh * extent + r) * D, m, x);
        }
    }
    if constexpr (kStage) {
        lds_barrier();
        // a pass of the block covers kRowBlock 16-byte vectors: whole runs
        // of kRowWaves rows of kRowBlock * 16 / (kRowWaves * D * 2) heads
        constexpr int VPR = D / VE;                  // vectors per head row
        constexpr int VPH = VPR * kRowWaves;         // vectors per head run
        constexpr int HPP = kRowBlock / VPH;         // heads per pass
        static_assert(HPP * VPH == kRowBlock, "whole head runs per pass");
        const int tr = (threadIdx.x % VPH) / VPR;    // row of the tile
        const int tv = threadIdx.x % VPR;            // vector in the row
        const int64_t rr = tile * kRowWaves + tr;
#pragma unroll
        for (int h0 = 0; h0 < NG * 4; h0 += HPP) {
            const int hh = h0 + threadIdx.x / VPH;
            if (hh < H && rr < extent) {
                const u32x4 o = *reinterpret_cast<const u32x4*>(&ost[tr][hh * D + tv * VE]);
                u32x4* dst = reinterpret_cast<u32x4*>(out + ((int64_t)hh * extent + rr) * D + tv * VE);
                if (T2H_NT) __builtin_nontemporal_store(o, dst); else *dst = o;
            }
        }
    }
}

// The v pass in the slab layout of the activation kernel: one 16-byte vector
// per thread. A wave covers 1 KB of one row's v (64 * V columns, i.e. 4
// heads of 128 f16), a block that piece for kVSlabRows consecutive rows, and
// consecutive blocks walk the pieces of a row tile (2-D grid: x = piece, y =
// row tile over lp). The piece's bias_v is read once per block into LDS
// behind an LDS-only barrier that leaves the row loads in flight. A vector
// lies inside one head (head_dim % V == 0) and lands at vh[h][r][d]; pad rows
// rows <= r < lp are zero. One vector per thread streams faster than the row
// wave's three (MI355X, 3 KB row pieces: ~81 % against ~71 % of HBM peak in
// the streaming probes).
constexpr int kVSlabRows = 4;
constexpr int kVSlabThreads = 64 * kVSlabRows;

struct PackVArgs {
    const void* v;      // [rows, H * D], rows in_stride apart
    void* vh;           // [H, lp, D]
    const float* bias;  // [H * D] or nullptr
    int64_t rows;
    int64_t lp;
    int64_t in_stride;
    int32_t cols;       // H * D
    int32_t dshift;     // log2(head_dim)
};

template <typename T, int V>
__global__ __launch_bounds__(kVSlabThreads) void pack_v_slab_kernel(PackVArgs a) {
    constexpr int Q = V / 4;   // float4 pieces of a lane's bias
    __shared__ float4 bl[64 * Q];   // the piece's bias in column order
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c0 = (int)blockIdx.x * (64 * V);   // < cols
    const int64_t r = (int64_t)blockIdx.y * kVSlabRows + wave;
    const int col = c0 + lane * V;
    const bool in_row = col < a.cols;
    const bool live = r < a.rows;
    const bool bias = a.bias != nullptr;   // block-uniform
    float4 bq;
    if (bias && wave < Q) {
        const int f = 4 * tid < a.cols - c0 ? c0 + 4 * tid : a.cols - 4;   // cols % 4 == 0
        bq = *reinterpret_cast<const float4*>(a.bias + f);
    }
    float v[V];
    if (a.rows > 0) {   // unconditional (clamped) row load; no rows at all: pads only
        const int64_t rl = live ? r : a.rows - 1;
        const int cl = in_row ? col : a.cols - V;
        load_elems<T, V, true>(static_cast<const T*>(a.v) + rl * a.in_stride + cl, v);
    }
    float b[V];
    if (bias) {
        if (wave < Q) bl[tid] = bq;
        lds_barrier();
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const float4 w = bl[lane * Q + q];
            b[4 * q] = w.x; b[4 * q + 1] = w.y; b[4 * q + 2] = w.z; b[4 * q + 3] = w.w;
        }
    }
    if (r >= a.lp || !in_row) return;
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = !live ? 0.0f : bias ? add_rn(v[i], b[i]) : v[i];
    const int h = col >> a.dshift;
    const int d = col - (h << a.dshift);
    store_elems<T, V, true>(static_cast<T*>(a.vh) + (((int64_t)h * a.lp + r) << a.dshift) + d, v);
}

// The v pass goes to pack_v_slab_kernel when its rows are 16-byte vectors
// of at least one slab; returns false when the row kernels must take it.
template <typename T>
bool v_slab_ok(const PackArgs& a) {
    constexpr int V = kPack<T>;
    const int64_t cols = (int64_t)a.heads * a.head_dim;
    return a.vh != nullptr && cols >= 64 * V && cols <= INT32_MAX - 64 * V && a.in_stride % V == 0 &&
           reinterpret_cast<uintptr_t>(a.v) % 16 == 0 && (a.lp + kVSlabRows - 1) / kVSlabRows < (int64_t(1) << 32);
}

template <typename T>
hipError_t launch_v_slab(const PackArgs& a, hipStream_t s) {
    constexpr int V = kPack<T>;
    const int32_t cols = a.heads * a.head_dim;
    const PackVArgs va{a.v, a.vh, a.bias_v, a.rows, a.lp, a.in_stride, cols, a.head_dim == 128 ? 7 : 6};
    const int64_t pieces = (cols + 64 * V - 1) / (64 * V);
    const int64_t tiles = (a.lp + kVSlabRows - 1) / kVSlabRows;
    hipLaunchKernelGGL((pack_v_slab_kernel<T, V>), dim3((unsigned)pieces, (unsigned)tiles), dim3(kVSlabThreads), 0, s,
                       va);
    return hipGetLastError();
}

// Heads per block: all of them when the row tiles alone fill the GPU,
// else the largest divisor of heads that still gives ~8 blocks per CU.
int heads_per_block(int64_t tiles, int tensors, int heads) {
    const int64_t want = 8LL * device_cu_count();
    int best = 1;
    for (int hpb = 1; hpb <= heads; ++hpb) {
        if (heads % hpb) continue;
        if (tiles * tensors * (heads / hpb) >= want || hpb == 1) best = hpb;
    }
    return best;
}

template <typename T, int D>
hipError_t launch_d(const PackArgs& a, const RopeSlots& tab, hipStream_t s) {
    const int64_t ext = a.mp > a.lp ? a.mp : a.lp;
    const int64_t tiles = (ext + kPackRows - 1) / kPackRows;
    PackOrder rows{};
    const bool v_slab = v_slab_ok<T>(a);
    if (a.qh != nullptr) rows.which[rows.n++] = 0;
    if (a.k_out != nullptr && !a.k_transposed) rows.which[rows.n++] = 1;
    if (a.vh != nullptr && !v_slab) rows.which[rows.n++] = 2;
    if (v_slab) {
        if (hipError_t e = launch_v_slab<T>(a, s); e != hipSuccess) return e;
    }
    if (rows.n > 0 && a.heads <= 16) {
        const int64_t blocks = (ext + kRowWaves - 1) / kRowWaves * rows.n;
        switch ((a.heads + 3) / 4) {
            case 1: hipLaunchKernelGGL((pack_rows_kernel<T, D, 1>), grid_1d(blocks), dim3(kRowBlock), 0, s, a, tab, rows); break;
            case 2: hipLaunchKernelGGL((pack_rows_kernel<T, D, 2>), grid_1d(blocks), dim3(kRowBlock), 0, s, a, tab, rows); break;
            case 3: hipLaunchKernelGGL((pack_rows_kernel<T, D, 3>), grid_1d(blocks), dim3(kRowBlock), 0, s, a, tab, rows); break;
            default: hipLaunchKernelGGL((pack_rows_kernel<T, D, 4>), grid_1d(blocks), dim3(kRowBlock), 0, s, a, tab, rows); break;
        }
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    } else if (rows.n > 0) {
        rows.hpb = heads_per_block(tiles, rows.n, a.heads);
        rows.groups = a.heads / rows.hpb;
        const int64_t blocks = tiles * rows.groups * rows.n;
        hipLaunchKernelGGL((pack_tile_kernel<T, D, false>), grid_1d(blocks), dim3(kPackBlock), 0, s, a, tab,
                           rows);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    if (a.k_out != nullptr && a.k_transposed) {
        PackOrder kt{};
        kt.n = 1;
        kt.which[0] = 1;
        kt.hpb = heads_per_block(tiles, 1, a.heads);
        kt.groups = a.heads / kt.hpb;
        hipLaunchKernelGGL((pack_tile_kernel<T, D, true>), grid_1d(tiles * kt.groups), dim3(kPackBlock), 0,
                           s, a, tab, kt);
        return hipGetLastError();
    }
    return hipSuccess;
}

template <typename T>
hipError_t launch_typed(const PackArgs& a, const RopeSlots& tab, hipStream_t s) {
    if (a.head_dim == 128) return launch_d<T, 128>(a, tab, s);
    return launch_d<T, 64>(a, tab, s);
}

}  // namespace

hipError_t launch_pack(const PackArgs& a, const RopeSlots& tab, hipStream_t s) {
    switch (a.dtype) {
        case T2H_F32: return launch_typed<float>(a, tab, s);
        case T2H_F16: return launch_typed<_Float16>(a, tab, s);
        default: return launch_typed<__bf16>(a, tab, s);
    }
}

}  // namespace t2h
