// Self-attention epilogue fused with the head-major packing of the attention
// operands: one pass over the qkv GEMM output instead of an in-place epilogue
// pass followed by two packing passes.
//
//   q, k, v [rows, H, D] (rows in_stride apart, e.g. views of a packed qkv
//   [rows, 3, H, D]) --(+bias, RMS q/k, RoPE q/k)-->
//   qh [H, mp, D] = q * 1/sqrt(D); k_out [H, D, lp] (transposed) or
//   [H, lp, D]; vh [H, lp, D]; pad rows rows..mp-1 / rows..lp-1 are zero.
//
// A block is 4 waves over a tile of 64 token rows x one head of one tensor.
// Each 16-lane DPP row of a wave holds one token row's head (lane m: elements
// [m*E, m*E+E), E = D/16), so a wave instruction covers 4 token rows and the
// per-head sum of squares is a 4-step DPP row sum; the head's bias and
// gamma * scale sit in registers for the whole tile. All 16 rows of a wave
// are loaded (clamped, unconditional) before any math. Row-major outputs are
// written straight from registers: a wave instruction writes 4 consecutive
// rows of one head, a contiguous span. The transposed k goes through LDS
// (64 x (D+1) f32, odd row pitch: conflict-free column reads) and leaves as
// 16-byte vectors along the token axis.
//
// Reference: gpu/attention.mojo:507-563 (bias_rms_rope_qkv), 566-594
// (pack_q_z), 634-662 (pack_kv_z), sequence 987-1013; cross chain q:
// 596-631 (bias_rms_q) + pack_q_z with stride H*D (sequence 1223-1234).
#include "t2h_device.h"
#include "t2h_internal.h"
#include "t2h_rope.h"

namespace t2h {
namespace {

constexpr int kPackRows = 64;
constexpr int kPackBlock = 256;
constexpr int kPackIters = kPackRows / 16;   // row groups of 4 per wave

// `order` maps blockIdx.z to the tensor a block packs: 0 = q, 1 = k, 2 = v.
struct PackOrder {
    int8_t which[3];
};

template <typename T, int D, bool KT>
__global__ __launch_bounds__(kPackBlock) void pack_tile_kernel(PackArgs a, RopeSlots tab, PackOrder order) {
    constexpr int E = D / 16;
    constexpr int P = E / 2;
    __shared__ float tile[KT ? kPackRows : 1][KT ? D + 1 : 1];
    const int lane = lane_id();
    const int g = lane >> 4;
    const int m = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int which = order.which[blockIdx.z];
    const int z = blockIdx.y;
    const int64_t t0 = (int64_t)blockIdx.x * kPackRows;
    const int64_t extent = which == 0 ? a.mp : a.lp;
    if (t0 >= extent) return;

    const T* __restrict__ in = static_cast<const T*>(which == 0 ? a.q : which == 1 ? a.k : a.v);
    const float* __restrict__ bias = which == 0 ? a.bias_q : which == 1 ? a.bias_k : a.bias_v;
    const float* __restrict__ gamma = which == 0 ? a.gamma_q : which == 1 ? a.gamma_k : nullptr;
    const bool rope = a.use_rope && which < 2;
    const int col = z * D + m * E;

    float v[kPackIters][E];
    if (a.rows > 0) {
#pragma unroll
        for (int it = 0; it < kPackIters; ++it) {
            const int64_t t = t0 + it * 16 + wave * 4 + g;
            const int64_t tl = t < a.rows ? t : a.rows - 1;
            load_elems<T, E, true>(in + tl * a.in_stride + col, v[it]);
        }
    } else {
#pragma unroll
        for (int it = 0; it < kPackIters; ++it)
#pragma unroll
            for (int i = 0; i < E; ++i) v[it][i] = 0.0f;
    }
    float bv[E], gv[E];
    if (bias != nullptr) load_params<E>(bias + col, bv);
    if (gamma != nullptr) {
        load_params<E>(gamma + col, gv);
#pragma unroll
        for (int i = 0; i < E; ++i) gv[i] *= a.rms_scale;
    }
    int ax[P];
    float fr[P];
    if (rope) {
#pragma unroll
        for (int j = 0; j < P; ++j) {
            ax[j] = tab.axis[m * P + j];
            fr[j] = tab.freq[m * P + j];
        }
    }
    const PosSource src{a.coords, a.coord_cols, a.grid_res, a.pos_dim};

#pragma unroll
    for (int it = 0; it < kPackIters; ++it) {
        const int64_t t = t0 + it * 16 + wave * 4 + g;
        const bool valid = t < a.rows;
        float* x = v[it];
        if (bias != nullptr) {
#pragma unroll
            for (int i = 0; i < E; ++i) x[i] = add_rn(x[i], bv[i]);
        }
        if (gamma != nullptr) {
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < E; ++i) ss += x[i] * x[i];
            ss = row16_sum(ss);
            const float rn = ss < 1e-24f ? 1e12f : __builtin_amdgcn_rsqf(ss);
#pragma unroll
            for (int i = 0; i < E; ++i) x[i] = (x[i] * rn) * gv[i];
        }
        if (rope) {
            const int64_t tv = valid ? t : 0;
            float pc[P], ps[P];
            if (a.phases != nullptr) {
                const int64_t l = tv % a.phase_rows;
                float tmp[2 * P];
                load_params<2 * P>(a.phases + (l * (D / 2) + m * P) * 2, tmp);
#pragma unroll
                for (int j = 0; j < P; ++j) { pc[j] = tmp[2 * j]; ps[j] = tmp[2 * j + 1]; }
            } else {
                float pos[T2H_MAX_POS_DIM];
                src.get(tv, pos);
#pragma unroll
                for (int j = 0; j < P; ++j) slot_phase(pos, ax[j], fr[j], pc[j], ps[j]);
            }
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const float re = x[2 * j], im = x[2 * j + 1];
                x[2 * j] = re * pc[j] - im * ps[j];
                x[2 * j + 1] = re * ps[j] + im * pc[j];
            }
        }
        if (which == 0) {
#pragma unroll
            for (int i = 0; i < E; ++i) x[i] = mul_rn(x[i], a.q_scale);
        }
        if (!valid) {
#pragma unroll
            for (int i = 0; i < E; ++i) x[i] = 0.0f;
        }
        if constexpr (KT) {
            const int tl = it * 16 + wave * 4 + g;
#pragma unroll
            for (int i = 0; i < E; ++i) tile[tl][m * E + i] = round_to<T>(x[i]);
        } else if (t < extent) {
            T* __restrict__ out = static_cast<T*>(which == 0 ? a.qh : which == 1 ? a.k_out : a.vh);
            store_elems<T, E, true>(out + ((int64_t)z * extent + t) * D + m * E, x);
        }
    }

    if constexpr (KT) {
        __syncthreads();
        constexpr int VE = kPack<T>;            // elements per 16-byte vector
        constexpr int VPR = kPackRows / VE;     // vectors per output row (one e)
        T* __restrict__ out = static_cast<T*>(a.k_out);
        for (int vi = threadIdx.x; vi < D * VPR; vi += kPackBlock) {
            const int e = vi / VPR;
            const int tq = (vi % VPR) * VE;
            if (t0 + tq >= extent) continue;
            float w[VE];
#pragma unroll
            for (int i = 0; i < VE; ++i) w[i] = tile[tq + i][e];
            store_elems<T, VE, true>(out + ((int64_t)z * D + e) * a.lp + t0 + tq, w);
        }
    }
}

template <typename T, int D>
hipError_t launch_d(const PackArgs& a, const RopeSlots& tab, hipStream_t s) {
    const int64_t ext = a.mp > a.lp ? a.mp : a.lp;
    const unsigned tiles = (unsigned)((ext + kPackRows - 1) / kPackRows);
    PackOrder rows{};
    int n = 0;
    if (a.qh != nullptr) rows.which[n++] = 0;
    if (a.k_out != nullptr && !a.k_transposed) rows.which[n++] = 1;
    if (a.vh != nullptr) rows.which[n++] = 2;
    if (n > 0) {
        hipLaunchKernelGGL((pack_tile_kernel<T, D, false>), dim3(tiles, a.heads, n), dim3(kPackBlock), 0, s, a, tab,
                           rows);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    if (a.k_out != nullptr && a.k_transposed) {
        PackOrder kt{};
        kt.which[0] = 1;
        hipLaunchKernelGGL((pack_tile_kernel<T, D, true>), dim3(tiles, a.heads, 1), dim3(kPackBlock), 0, s, a, tab,
                           kt);
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
