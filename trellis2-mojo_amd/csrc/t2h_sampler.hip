// One flow-matching Euler step of the sampler over a flat state x_t:
// classifier-free-guidance combine, optional CFG rescale, the Euler update and
// the x_0 prediction, in one elementwise pass (plus, for the rescale, a
// statistics pass and a per-segment ratio).
//
//   pred   = v_pos (no guidance) or fl(v_pos * f32(g)) + fl(v_neg * f32(1-g))
//   rescale (guidance_rescale > 0):
//     x0_pos = fl(x*a) - fl(v_pos*cc), x0_cfg = fl(x*a) - fl(pred*cc)
//     ratio[s] = std(x0_pos) / std(x0_cfg) over segment s
//     pred = (fl(a*x) - (fl(gr*fl(x0_cfg*ratio)) + fl((1-gr)*x0_cfg))) / cc
//   x_prev  = fl(x - fl(pred * f32(t - t_prev)))
//   pred_x0 = fl(x*a) - fl(pred*cc)
// with a = f32(1 - sigma_min), cc = f32(sigma_min + (1 - sigma_min) t).
// Segments are rows of row_size elements (dense state, unbiased std) or the
// caller's token segments (varlen state, biased std). The statistics are
// summed in f64 per block of kChunk elements, then per segment in a fixed
// order, so the result is deterministic.
//
// Reference: samplers/flow_euler.mojo:56-57 (_scaled), 68-70
// (_v_to_xstart), 75-149 (_rescale_pred), 151-181 (_inference),
// 196-210 (_sample_impl step).
#include "t2h_device.h"
#include "t2h_internal.h"

namespace t2h {
namespace {

constexpr int kEulerBlock = 256;

// Segment bounds of block b: blocks tile every segment in kEulerChunk pieces.
struct SegMap {
    __device__ __forceinline__ static void locate(const EulerArgs& a, int64_t b, int& s, int64_t& lo, int64_t& hi) {
        if (a.uniform) {
            const int64_t nb = (a.row_size + kEulerChunk - 1) / kEulerChunk;
            s = (int)(b / nb);
            const int64_t j = b % nb;
            lo = s * a.row_size + j * kEulerChunk;
            hi = min(lo + kEulerChunk, (s + 1) * a.row_size);
        } else {
            s = 0;
            while (s + 1 < a.nseg && a.blk_base[s + 1] <= b) ++s;
            const int64_t j = b - a.blk_base[s];
            lo = a.bounds[s] + j * kEulerChunk;
            hi = min(lo + kEulerChunk, a.bounds[s + 1]);
        }
    }
};

template <typename T>
__device__ __forceinline__ float cfg_pred(const EulerArgs& a, int64_t e, float& pos) {
    pos = ld1(static_cast<const T*>(a.v_pos) + e);
    if (a.mode == 0) return pos;
    const float neg = ld1(static_cast<const T*>(a.v_neg) + e);
    return add_rn(mul_rn(pos, a.gp), mul_rn(neg, a.gn));
}

__device__ __forceinline__ float v_to_x0(float x, float v, float a, float cc) {
    return sub_rn(mul_rn(x, a), mul_rn(v, cc));
}

// f64 block sum of 4 values through LDS, result in thread 0.
__device__ __forceinline__ void block_sum4(double (&v)[4], double (*sh)[4]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < 4; ++k) sh[t][k] = v[k];
    __syncthreads();
    for (int w = kEulerBlock / 2; w > 0; w >>= 1) {
        if (t < w) {
#pragma unroll
            for (int k = 0; k < 4; ++k) sh[t][k] += sh[t + w][k];
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = sh[0][k];
}

template <typename T>
__global__ __launch_bounds__(kEulerBlock) void euler_stats_kernel(EulerArgs a) {
    __shared__ double sh[kEulerBlock][4];
    const int64_t b = block_linear();
    if (b >= a.nblocks) return;
    int s;
    int64_t lo, hi;
    SegMap::locate(a, b, s, lo, hi);
    const T* __restrict__ x = static_cast<const T*>(a.x);
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int64_t e = lo + threadIdx.x; e < hi; e += kEulerBlock) {
        float pos;
        const float pred = cfg_pred<T>(a, e, pos);
        const float xv = ld1(x + e);
        const double x0p = v_to_x0(xv, pos, a.a, a.cc);
        const double x0c = v_to_x0(xv, pred, a.a, a.cc);
        acc[0] += x0p;
        acc[1] += x0p * x0p;
        acc[2] += x0c;
        acc[3] += x0c * x0c;
    }
    block_sum4(acc, sh);
    if (threadIdx.x == 0) {
        double* p = a.partial + b * 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) p[k] = acc[k];
    }
}

// One block per segment: fixed-order sum of the segment's block partials.
__global__ __launch_bounds__(kEulerBlock) void euler_ratio_kernel(EulerArgs a) {
    __shared__ double sh[kEulerBlock][4];
    const int64_t sl = block_linear();
    if (sl >= a.nseg) return;
    const int s = (int)sl;
    int64_t b0, b1, m;
    if (a.uniform) {
        const int64_t nb = (a.row_size + kEulerChunk - 1) / kEulerChunk;
        b0 = s * nb;
        b1 = b0 + nb;
        m = a.row_size;
    } else {
        b0 = a.blk_base[s];
        b1 = a.blk_base[s + 1];
        m = a.bounds[s + 1] - a.bounds[s];
    }
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int64_t b = b0 + threadIdx.x; b < b1; b += kEulerBlock) {
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] += a.partial[b * 4 + k];
    }
    block_sum4(acc, sh);
    if (threadIdx.x == 0) {
        const double md = (double)m;
        double vp, vc;
        if (a.uniform) {   // unbiased, one segment per row
            vp = (acc[1] - acc[0] * (acc[0] / md)) / (md - 1.0);
            vc = (acc[3] - acc[2] * (acc[2] / md)) / (md - 1.0);
        } else {           // biased: mean(x^2) - mean(x)^2
            vp = acc[1] / md - (acc[0] / md) * (acc[0] / md);
            vc = acc[3] / md - (acc[2] / md) * (acc[2] / md);
        }
        a.ratio[s] = m > 0 ? (float)(sqrt(vp > 0.0 ? vp : 0.0) / sqrt(vc > 0.0 ? vc : 0.0)) : 0.0f;
        if (a.uniform && m == 1) a.ratio[s] = __builtin_nanf("");   // 0/0 as the reference's m - 1 = 0
    }
}

template <typename T>
__global__ __launch_bounds__(kEulerBlock) void euler_apply_kernel(EulerArgs a) {
    const T* __restrict__ x = static_cast<const T*>(a.x);
    T* __restrict__ xp = static_cast<T*>(a.x_prev);
    T* __restrict__ x0o = static_cast<T*>(a.pred_x0);
    const int64_t b = block_linear();
    if (b >= a.nblocks) return;
    int s = 0;
    int64_t lo, hi;
    if (a.mode == 2) {
        SegMap::locate(a, b, s, lo, hi);
    } else {
        lo = b * kEulerChunkPlain;
        hi = min(lo + kEulerChunkPlain, a.n);
    }
    const float ratio = a.mode == 2 ? a.ratio[s] : 0.0f;
    for (int64_t e = lo + threadIdx.x; e < hi; e += kEulerBlock) {
        const float xv = ld1(x + e);
        float pos;
        float pred = cfg_pred<T>(a, e, pos);
        if (a.mode == 2) {
            const float x0c = v_to_x0(xv, pred, a.a, a.cc);
            const float x0r = mul_rn(x0c, ratio);
            const float x0 = add_rn(mul_rn(a.gr, x0r), mul_rn(a.one_m_gr, x0c));
            pred = __fdiv_rn(sub_rn(mul_rn(a.a, xv), x0), a.cc);
        }
        st1(xp + e, sub_rn(xv, mul_rn(pred, a.dt)));
        if (x0o != nullptr) st1(x0o + e, v_to_x0(xv, pred, a.a, a.cc));
    }
}

// Rows outside every varlen segment: the reference's rescale leaves their
// prediction at zero, so x_prev = x and pred_x0 = fl(x * a).
template <typename T>
__global__ __launch_bounds__(kEulerBlock) void euler_uncovered_kernel(EulerArgs a, int64_t lo, int64_t hi) {
    const T* __restrict__ x = static_cast<const T*>(a.x);
    T* __restrict__ xp = static_cast<T*>(a.x_prev);
    T* __restrict__ x0o = static_cast<T*>(a.pred_x0);
    for (int64_t e = lo + (int64_t)blockIdx.x * kEulerBlock + threadIdx.x; e < hi;
         e += (int64_t)gridDim.x * kEulerBlock) {
        const float xv = ld1(x + e);
        st1(xp + e, sub_rn(xv, mul_rn(0.0f, a.dt)));
        if (x0o != nullptr) st1(x0o + e, v_to_x0(xv, 0.0f, a.a, a.cc));
    }
}

template <typename T>
hipError_t launch_typed(const EulerArgs& a, int64_t blocks, int64_t cover_lo, int64_t cover_hi, hipStream_t st) {
    if (a.mode == 2) {
        if (blocks > 0) {
            hipLaunchKernelGGL(euler_stats_kernel<T>, grid_1d(blocks), dim3(kEulerBlock), 0, st, a);
            hipLaunchKernelGGL(euler_ratio_kernel, grid_1d(a.nseg), dim3(kEulerBlock), 0, st, a);
            hipLaunchKernelGGL(euler_apply_kernel<T>, grid_1d(blocks), dim3(kEulerBlock), 0, st, a);
        }
        if (cover_lo > 0) {
            const int64_t g = (cover_lo + kEulerBlock - 1) / kEulerBlock;
            hipLaunchKernelGGL(euler_uncovered_kernel<T>, dim3((unsigned)(g < 4096 ? g : 4096)), dim3(kEulerBlock),
                               0, st, a, (int64_t)0, cover_lo);
        }
        if (cover_hi < a.n) {
            const int64_t g = (a.n - cover_hi + kEulerBlock - 1) / kEulerBlock;
            hipLaunchKernelGGL(euler_uncovered_kernel<T>, dim3((unsigned)(g < 4096 ? g : 4096)), dim3(kEulerBlock),
                               0, st, a, cover_hi, a.n);
        }
    } else {
        hipLaunchKernelGGL(euler_apply_kernel<T>, grid_1d(a.nblocks), dim3(kEulerBlock), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_euler(const EulerArgs& a, int64_t blocks, int64_t cover_lo, int64_t cover_hi, hipStream_t s) {
    switch (a.dtype) {
        case T2H_F32: return launch_typed<float>(a, blocks, cover_lo, cover_hi, s);
        case T2H_F16: return launch_typed<_Float16>(a, blocks, cover_lo, cover_hi, s);
        default: return launch_typed<__bf16>(a, blocks, cover_lo, cover_hi, s);
    }
}

}  // namespace t2h
