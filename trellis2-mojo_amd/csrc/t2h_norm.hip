// LayerNorm + adaLN epilogue over token rows, and the fused gated-residual
// join + LayerNorm (one HBM pass for `x += gate*(h+bias); y = LN(x)*(1+scale)+shift`).
//
// Fast path: one wave64 per row, the row held in VGPRs (C = 64 * NCH * E with
// E = 16 B of storage per lane, e.g. C = 1536: f32 NCH 6, f16/bf16 NCH 3), so
// the two-pass mean/variance never re-reads HBM. A block is 8 rows, one wave
// each, on a non-persistent grid (many short blocks stream HBM better on
// MI355X than persistent waves). Each wave issues its row loads first; the
// block then stages the parameter rows of its first row's batch in LDS
// behind an LDS-only barrier, so the epilogue never waits on L2. Reductions
// are DPP row sums plus four readlanes. Every output element follows the reference's f32
// rounding sequence; only the order of the two row sums differs from the
// reference.
//
// Reference: modules/nn.mojo:314-369 (LayerNorm32), 660-689 (modulate),
// sparse/transformer/modulated.mojo:60-65 (gathered modulate),
// gpu/block.mojo:47-110 (ln_mod_rows, gate_add_bias_rows).
#include "t2h_device.h"
#include "t2h_internal.h"

namespace t2h {
namespace {

#ifndef T2H_LN_WAVES
#define T2H_LN_WAVES 8
#endif
constexpr int kWavesPerBlock = T2H_LN_WAVES;   // fast path: rows per block
constexpr int kFastBlock = 64 * kWavesPerBlock;
constexpr int kBlock = 256;                      // generic path


// y = LN epilogue of one centred value d = x - mean (f32), in the reference's
// order: n = d * inv_std, then n * (1 + scale) + shift (pb holds the already
// rounded 1 + scale) or n * w + b.
__device__ __forceinline__ float ln_epilogue(float d, float inv, int mode, float pa, float pb) {
    const float n = mul_rn(d, inv);
    if (mode == T2H_LN_MODULATE) return add_rn(mul_rn(n, pb), pa);
    if (mode == T2H_LN_AFFINE) return add_rn(mul_rn(n, pa), pb);
    return n;
}

// E f32 values from LDS (E a multiple of 4, 16-byte aligned).
template <int E>
__device__ __forceinline__ void lds_params(const float* p, float* f) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int c4 = 0; c4 < E / 4; ++c4) {
        const float4 w = q[c4];
        f[4 * c4] = w.x; f[4 * c4 + 1] = w.y; f[4 * c4 + 2] = w.z; f[4 * c4 + 3] = w.w;
    }
}

template <typename T, int NCH, bool JOIN>
__global__ __launch_bounds__(kFastBlock) void ln_rows_kernel(LnArgs a) {
    constexpr int E = kPack<T>;
    constexpr int C = 64 * NCH * E;
    constexpr int NP = JOIN ? 4 : 2;   // staged parameter rows: p0, p1 [, bias, gate]
    __shared__ __attribute__((aligned(16))) float ps[NP * C];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r0 = front_of(block_linear(), a.fper) * kWavesPerBlock;
    if (r0 >= a.rows) return;   // past the last row of a 2-D grid (block-uniform)
    const int64_t r = r0 + wave;
    const bool live = r < a.rows;
    const int64_t rl = live ? r : a.rows - 1;   // dead waves load a valid row, store nothing
    const T* x = static_cast<const T*>(a.x);   // may alias x_out: no __restrict__
    const T* __restrict__ h = static_cast<const T*>(a.h);
    T* xo = static_cast<T*>(a.x_out);
    T* __restrict__ yo = static_cast<T*>(a.y_out);
    const int64_t base = rl * (int64_t)C;

    // 1. the row loads, all in flight before anything else
    float v[NCH][E];
    float hv[NCH][E];
    // large launches: x's first 1 KB piece with the default cache policy,
    // the rest (h's pieces included: one cached load of six measured faster
    // than two) non-temporal; a buffer load, not merged with its
    // non-temporal twins
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if (c == 0 && a.cached) {
            load_elems_cached<T, E>(x + base, (c * 64 + lane) * E, C, v[c]);
            if (JOIN) load_elems<T, E, true>(h + base + (c * 64 + lane) * E, hv[c]);
        } else {
            load_elems<T, E, true>(x + base + (c * 64 + lane) * E, v[c]);
            if (JOIN) load_elems<T, E, true>(h + base + (c * 64 + lane) * E, hv[c]);
        }
    }

    // 2. stage the parameter rows of the block's first row's batch in LDS
    //    (modulate: shift and the rounded 1 + scale; affine: weight, bias;
    //    join: bias and gate rows)
    const bool need_b = a.mode == T2H_LN_MODULATE || (JOIN && a.gate);
    const BatchMap bm{a.batch.offsets, a.batch.rows_per_batch, a.batch.nbatch};
    const int32_t b0 = need_b ? bm.batch_of(r0) : 0;
    const int64_t prow = a.mode == T2H_LN_MODULATE ? b0 * a.p_stride : 0;
    for (int i = threadIdx.x * 4; i < C; i += kFastBlock * 4) {
        float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
        if (a.mode != T2H_LN_PLAIN) {
            w0 = *reinterpret_cast<const float4*>(a.p0 + prow + i);
            w1 = *reinterpret_cast<const float4*>(a.p1 + prow + i);
            if (a.mode == T2H_LN_MODULATE) {
                w1.x = add_rn(1.0f, w1.x); w1.y = add_rn(1.0f, w1.y);
                w1.z = add_rn(1.0f, w1.z); w1.w = add_rn(1.0f, w1.w);
            }
        }
        *reinterpret_cast<float4*>(&ps[i]) = w0;
        *reinterpret_cast<float4*>(&ps[C + i]) = w1;
        if (JOIN) {
            if (a.bias) *reinterpret_cast<float4*>(&ps[2 * C + i]) = *reinterpret_cast<const float4*>(a.bias + i);
            if (a.gate)
                *reinterpret_cast<float4*>(&ps[3 * C + i]) =
                    *reinterpret_cast<const float4*>(a.gate + b0 * a.gate_stride + i);
        }
    }
    // LDS-only barrier: lgkmcnt(0) covers this wave's LDS (and scalar) traffic;
    // the row loads (vmcnt) stay in flight across it.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (!live) return;

    // rows of another batch than the block's first (only at batch
    // boundaries) read their per-batch rows (modulate shift/scale, gate) from
    // global memory; the affine weight/bias and the join bias are per channel
    // and always come from LDS
    const int32_t b = need_b ? bm.batch_of(r) : 0;
    const bool staged = b == b0;

    if (JOIN) {   // x_out = x + fl(fl(h + bias) * gate[b]), as stored in T
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int col = (c * 64 + lane) * E;
            float jb[E], jg[E];
            if (a.bias) lds_params<E>(&ps[2 * C + col], jb);
            if (a.gate) {
                if (staged) lds_params<E>(&ps[3 * C + col], jg);
                else load_params<E>(a.gate + b * a.gate_stride + col, jg);
            }
#pragma unroll
            for (int i = 0; i < E; ++i) {
                float t = a.bias ? add_rn(hv[c][i], jb[i]) : hv[c][i];
                if (a.gate) t = mul_rn(t, jg[i]);
                v[c][i] = round_to<T>(add_rn(v[c][i], t));
            }
            store_elems<T, E, true>(xo + base + col, v[c]);
        }
    }

    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int i = 0; i < E; ++i) s += v[c][i];
    const float mean = wave_sum(s) / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int i = 0; i < E; ++i) {
            v[c][i] = sub_rn(v[c][i], mean);   // keep x - mean for the epilogue
            q += v[c][i] * v[c][i];
        }
    const float var = wave_sum(q) / (float)C;
    const float inv = 1.0f / sqrtf(var + a.eps);

#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = (c * 64 + lane) * E;
        float pa[E], pb[E];
        if (a.mode != T2H_LN_MODULATE || staged) {
            lds_params<E>(&ps[col], pa);
            lds_params<E>(&ps[C + col], pb);
        } else {
            load_params<E>(a.p0 + b * a.p_stride + col, pa);
            load_params<E>(a.p1 + b * a.p_stride + col, pb);
#pragma unroll
            for (int i = 0; i < E; ++i) pb[i] = add_rn(1.0f, pb[i]);   // 1 + scale
        }
        float y[E];
#pragma unroll
        for (int i = 0; i < E; ++i) y[i] = ln_epilogue(v[c][i], inv, a.mode, pa[i], pb[i]);
        store_elems<T, E, true>(yo + base + col, y);
    }
}

// Any cols: one 256-thread block per row (grid-stride), block reduction
// through LDS, values re-read from memory for each pass. With JOIN, pass 1
// writes x_out and passes 2 and 3 read the stored (already rounded) value
// back: x_out may alias x, so recomputing x + gate*h from x would add the
// gated term twice. Each thread reads back only the elements it wrote.
template <typename T, bool JOIN>
__global__ __launch_bounds__(kBlock) void ln_rows_generic(LnArgs a) {
    __shared__ float red[kWavesPerBlock];
    const T* x = static_cast<const T*>(a.x);   // may alias x_out: no __restrict__
    const T* __restrict__ h = static_cast<const T*>(a.h);
    T* xo = static_cast<T*>(a.x_out);
    T* __restrict__ yo = static_cast<T*>(a.y_out);
    const BatchMap bm{a.batch.offsets, a.batch.rows_per_batch, a.batch.nbatch};
    const int C = a.cols;
    const int tid = threadIdx.x, wid = tid >> 6;

    auto block_sum = [&](float v) -> float {
        v = wave_sum(v);
        __syncthreads();
        if ((tid & 63) == 0) red[wid] = v;
        __syncthreads();
        return (red[0] + red[1]) + (red[2] + red[3]);
    };

    for (int64_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
        const int64_t base = r * (int64_t)C;
        const int32_t b = (a.mode == T2H_LN_MODULATE || (JOIN && a.gate)) ? bm.batch_of(r) : 0;
        auto joined = [&](int c) -> float {   // pass 1: x + fl(fl(h + bias) * gate), rounded to T
            float xv = ld1(x + base + c);
            if (JOIN) {
                float t = ld1(h + base + c);
                if (a.bias) t = add_rn(t, a.bias[c]);
                if (a.gate) t = mul_rn(t, a.gate[b * a.gate_stride + c]);
                xv = round_to<T>(add_rn(xv, t));
            }
            return xv;
        };
        auto value = [&](int c) -> float {    // passes 2 and 3: the row as pass 1 left it
            return JOIN ? ld1(xo + base + c) : ld1(x + base + c);
        };
        float s = 0.0f;
        for (int c = tid; c < C; c += kBlock) {
            const float xv = joined(c);
            if (JOIN) st1(xo + base + c, xv);
            s += xv;
        }
        const float mean = block_sum(s) / (float)C;
        float q = 0.0f;
        for (int c = tid; c < C; c += kBlock) {
            const float d = sub_rn(value(c), mean);
            q += d * d;
        }
        const float var = block_sum(q) / (float)C;
        const float inv = 1.0f / sqrtf(var + a.eps);
        const int32_t pbx = (a.mode == T2H_LN_MODULATE) ? b : 0;
        for (int c = tid; c < C; c += kBlock) {
            const float pa = a.mode != T2H_LN_PLAIN ? a.p0[pbx * a.p_stride + c] : 0.0f;
            float pb = a.mode != T2H_LN_PLAIN ? a.p1[pbx * a.p_stride + c] : 0.0f;
            if (a.mode == T2H_LN_MODULATE) pb = add_rn(1.0f, pb);
            st1(yo + base + c, ln_epilogue(sub_rn(value(c), mean), inv, a.mode, pa, pb));
        }
    }
}

template <typename K>
int resident_blocks(K kernel) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, kBlock, 0) != hipSuccess || nb <= 0) nb = 2;
    return nb * device_cu_count();
}

template <typename T, int NCH, bool JOIN>
hipError_t launch_fast(LnArgs a, hipStream_t s) {
    const int64_t grid = (a.rows + kWavesPerBlock - 1) / kWavesPerBlock;
    a.fper = front_per(grid);
    a.cached = a.rows * (int64_t)a.cols * (int64_t)sizeof(T) * (JOIN ? 4 : 2) >= T2H_CACHED_SHARE_MIN;
    hipLaunchKernelGGL((ln_rows_kernel<T, NCH, JOIN>), grid_1d(front_grid(grid)), dim3(kFastBlock), 0, s, a);
    return hipGetLastError();
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T, bool JOIN>
hipError_t launch_typed(const LnArgs& a, hipStream_t s) {
    constexpr int E = kPack<T>;
    const bool aligned = al16(a.x) && al16(a.h) && al16(a.x_out) && al16(a.y_out) && al16(a.p0) &&
                         al16(a.p1) && al16(a.bias) && al16(a.gate) && (a.p_stride % 4 == 0) &&
                         (a.gate_stride % 4 == 0);
    if (aligned && a.cols % (64 * E) == 0) {
        switch (a.cols / (64 * E)) {
            case 1: return launch_fast<T, 1, JOIN>(a, s);
            case 2: return launch_fast<T, 2, JOIN>(a, s);
            case 3: return launch_fast<T, 3, JOIN>(a, s);
            case 4: return launch_fast<T, 4, JOIN>(a, s);
            case 6: return launch_fast<T, 6, JOIN>(a, s);
            case 8: return launch_fast<T, 8, JOIN>(a, s);
            default: break;
        }
    }
    auto k = ln_rows_generic<T, JOIN>;
    static const int cap = resident_blocks(k);
    const int grid = (int)(a.rows < cap ? a.rows : cap);
    hipLaunchKernelGGL(k, dim3(grid), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

template <bool JOIN>
hipError_t launch_join(const LnArgs& a, hipStream_t s) {
    switch (a.dtype) {
        case T2H_F32: return launch_typed<float, JOIN>(a, s);
        case T2H_F16: return launch_typed<_Float16, JOIN>(a, s);
        default: return launch_typed<__bf16, JOIN>(a, s);
    }
}

}  // namespace

hipError_t launch_ln(const LnArgs& a, hipStream_t s) {
    return a.h ? launch_join<true>(a, s) : launch_join<false>(a, s);
}

}  // namespace t2h
