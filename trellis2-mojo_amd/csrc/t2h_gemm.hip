// Weight GEMM on the gfx950 matrix cores with the per-token epilogue in its
// store:
//
//   acc[t, n] = sum_k x[t, k] * w[n, k]        (f16 or bf16 operands, f32 sums)
//   out[t, n] = act(acc[t, n] + bias[n])        (t2h_linear)
//
// x is the token rows [rows, K] and w a linear's weight in its checkpoint
// layout [N, K]; both are K-contiguous, which is what the MFMA operands read.
// The weight rows are the MFMA's A operand and the token rows its B operand,
// so a 32x32 MFMA tile is 32 features x 32 tokens and each lane's 16
// accumulators hold one token (lane % 32) and four runs of four consecutive
// features (rows 8q + 4(lane / 32) + 0..3, q = 0..3). Consecutive features in
// one lane keep a RoPE pair (2p, 2p + 1) and a 16-byte store together; the
// two lanes l and l ^ 32 hold the two halves of every 8-feature group.
//
// Products of two f16 (or bf16) values are exact in f32 and the sums are f32,
// as in the reference's 16-bit-weight kernel gemm_tiled_f16sh (both operands
// rounded to f16, f32 accumulation; gpu/linear.mojo:326-388, selected by
// GpuLinear.try_build 430-465); only the summation order differs.
//
// Tiling: a block of 4 waves computes 256 features x 128 tokens (2 x 2 waves
// of 128 x 64, 8 MFMA tiles and 128 accumulators per lane). K advances in
// steps of 32 through double-buffered LDS tiles whose rows are padded by 16
// bytes (conflict-free 16-byte fragment reads); the next step's global loads
// are in flight while the current step's MFMAs run. Tiles are numbered
// token-tile major and the numbers are dealt to the 8 XCDs in contiguous
// ranges, so the feature tiles of one token tile run on one XCD one after
// the other and read its x rows from that XCD's L2.
//
// Reference: GpuLinear.enqueue_gemm (gpu/linear.mojo:535-560, c[m, co] =
// a[m, ci] @ W^T), the MLP's lin0 + gelu_tanh_bias (gpu/linear.mojo:662-684,
// 776-809).
#include "t2h_device.h"
#include "t2h_internal.h"
#include "t2h_act.h"

namespace t2h {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<_Float16> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    __device__ static __forceinline__ f32x16 run(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<__bf16> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    __device__ static __forceinline__ f32x16 run(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

#ifndef T2H_GEMM_BK
#define T2H_GEMM_BK 32
#endif
constexpr int kGemmThreads = 256;
constexpr int kBF = 256;              // features per block
constexpr int kBT = 128;              // tokens per block
constexpr int kBK = T2H_GEMM_BK;      // k per LDS stage
constexpr int kWF = kBF / 2;          // features per wave
constexpr int kWT = kBT / 2;          // tokens per wave
constexpr int kFI = kWF / 32;         // MFMA tiles along features
constexpr int kTJ = kWT / 32;         // MFMA tiles along tokens
constexpr int kStr = kBK + 8;         // LDS row pitch in elements (+16 bytes)
constexpr int kCpr = kBK / 8;         // 16-byte chunks per tile row
constexpr int kLA = kBF * kCpr / kGemmThreads;   // weight chunks per thread per stage
constexpr int kLB = kBT * kCpr / kGemmThreads;   // token chunks per thread per stage
static_assert(kLA >= 1 && kLB >= 1, "tile too small for the block");

// Tile u of nb, dealt so that XCD x (blocks b with b % 8 == x) takes the
// contiguous range of tiles [x*q + min(x, r), ...): a bijection of [0, nb).
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t nb) {
    const int64_t q = nb >> 3, r = nb & 7, x = b & 7, k = b >> 3;
    return x * q + (x < r ? x : r) + k;
}

// One token of the epilogue: four consecutive features starting at feature
// n, as f32 values after bias and activation, stored to out row t.
template <typename O>
__device__ __forceinline__ void store4(O* p, const float* v) {
    store_elems<O, 4>(p, v);
}

template <int ACT>
__device__ __forceinline__ float epi_f(float acc, float b) {
    const float v = bias_add(acc, b);
    if constexpr (ACT < 0) return v;
    else return act_f<ACT>(v);
}

template <typename T, typename O, int ACT>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs a) {
    using V8 = typename Mfma<T>::v8;
    __shared__ __attribute__((aligned(16))) T sa[2][kBF * kStr];
    __shared__ __attribute__((aligned(16))) T sb[2][kBT * kStr];

    const int64_t b = block_linear();
    if (b >= a.nblocks) return;
    const int64_t u = xcd_tile(b, a.nblocks);
    const int64_t tt = u / a.ftiles;
    const int ft = (int)(u - tt * a.ftiles);
    const int64_t t0 = tt * kBT;
    const int64_t n0 = (int64_t)ft * kBF;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wf = wave & 1;
    const int wt = wave >> 1;

    const T* __restrict__ x = static_cast<const T*>(a.x);
    const T* __restrict__ w = static_cast<const T*>(a.w);
    const int64_t last = a.rows - 1;

    // this thread's 16-byte chunks of each stage: source and LDS offset
    const T* ga[kLA];
    int la[kLA];
#pragma unroll
    for (int i = 0; i < kLA; ++i) {
        const int c = tid + i * kGemmThreads;
        const int row = c / kCpr, kc = c % kCpr;
        ga[i] = w + (n0 + row) * (int64_t)a.k + kc * 8;
        la[i] = row * kStr + kc * 8;
    }
    const T* gb[kLB];
    int lb[kLB];
#pragma unroll
    for (int i = 0; i < kLB; ++i) {
        const int c = tid + i * kGemmThreads;
        const int row = c / kCpr, kc = c % kCpr;
        const int64_t t = t0 + row < last ? t0 + row : last;   // pad tokens read the last row
        gb[i] = x + t * a.ldx + kc * 8;
        lb[i] = row * kStr + kc * 8;
    }

    u32x4 ra[kLA], rb[kLB];
#pragma unroll
    for (int i = 0; i < kLA; ++i) ra[i] = *reinterpret_cast<const u32x4*>(ga[i]);
#pragma unroll
    for (int i = 0; i < kLB; ++i) rb[i] = *reinterpret_cast<const u32x4*>(gb[i]);
#pragma unroll
    for (int i = 0; i < kLA; ++i) *reinterpret_cast<u32x4*>(&sa[0][la[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < kLB; ++i) *reinterpret_cast<u32x4*>(&sb[0][lb[i]]) = rb[i];
    __syncthreads();

    f32x16 acc[kFI][kTJ];
#pragma unroll
    for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
        for (int tj = 0; tj < kTJ; ++tj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fi][tj][r] = 0.0f;

    // fragment read offsets: row lane % 32 of each MFMA tile, k half lane / 32
    const int fa = (wf * kWF + (lane & 31)) * kStr + (lane >> 5) * 8;
    const int fb = (wt * kWT + (lane & 31)) * kStr + (lane >> 5) * 8;

    const int ksteps = a.k / kBK;
    for (int ks = 0; ks < ksteps; ++ks) {
        const int cur = ks & 1;
        const bool more = ks + 1 < ksteps;
        if (more) {
            const int64_t ko = (int64_t)(ks + 1) * kBK;
#pragma unroll
            for (int i = 0; i < kLA; ++i) ra[i] = *reinterpret_cast<const u32x4*>(ga[i] + ko);
#pragma unroll
            for (int i = 0; i < kLB; ++i) rb[i] = *reinterpret_cast<const u32x4*>(gb[i] + ko);
        }
#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
            V8 af[kFI], bf[kTJ];
#pragma unroll
            for (int fi = 0; fi < kFI; ++fi)
                af[fi] = *reinterpret_cast<const V8*>(&sa[cur][fa + fi * 32 * kStr + s * 16]);
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj)
                bf[tj] = *reinterpret_cast<const V8*>(&sb[cur][fb + tj * 32 * kStr + s * 16]);
#pragma unroll
            for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
                for (int tj = 0; tj < kTJ; ++tj) acc[fi][tj] = Mfma<T>::run(af[fi], bf[tj], acc[fi][tj]);
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < kLA; ++i) *reinterpret_cast<u32x4*>(&sa[cur ^ 1][la[i]]) = ra[i];
#pragma unroll
            for (int i = 0; i < kLB; ++i) *reinterpret_cast<u32x4*>(&sb[cur ^ 1][lb[i]]) = rb[i];
        }
        __syncthreads();
    }

    // epilogue: lane holds token t of each token tile and features
    // n + 8q + 4(lane / 32) + 0..3 of each feature tile
    O* __restrict__ out = static_cast<O*>(a.out);
    const int half = lane >> 5;
#pragma unroll
    for (int tj = 0; tj < kTJ; ++tj) {
        const int64_t t = t0 + wt * kWT + tj * 32 + (lane & 31);
        if (t >= a.rows) continue;
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t n = n0 + wf * kWF + fi * 32 + q * 8 + half * 4;
                float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (a.bias != nullptr) load_params<4>(a.bias + n, bv);
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = epi_f<ACT>(acc[fi][tj][q * 4 + i], bv[i]);
                store4<O>(out + t * a.ldo + n, v);
            }
        }
    }
}

template <typename T, typename O>
hipError_t gemm_act(const GemmArgs& a, hipStream_t s) {
    const dim3 g = grid_1d(a.nblocks), blk(kGemmThreads);
    switch (a.act) {
        case T2H_ACT_RELU: hipLaunchKernelGGL((gemm_kernel<T, O, T2H_ACT_RELU>), g, blk, 0, s, a); break;
        case T2H_ACT_SILU: hipLaunchKernelGGL((gemm_kernel<T, O, T2H_ACT_SILU>), g, blk, 0, s, a); break;
        case T2H_ACT_GELU: hipLaunchKernelGGL((gemm_kernel<T, O, T2H_ACT_GELU>), g, blk, 0, s, a); break;
        case T2H_ACT_GELU_TANH: hipLaunchKernelGGL((gemm_kernel<T, O, T2H_ACT_GELU_TANH>), g, blk, 0, s, a); break;
        default: hipLaunchKernelGGL((gemm_kernel<T, O, -1>), g, blk, 0, s, a); break;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t gemm_typed(const GemmArgs& a, hipStream_t s) {
    if (a.out_dtype == T2H_F32) return gemm_act<T, float>(a, s);
    return gemm_act<T, T>(a, s);
}

}  // namespace

int32_t gemm_feature_tile() { return kBF; }
int32_t gemm_k_step() { return kBK; }

hipError_t launch_gemm(GemmArgs a, hipStream_t s) {
    a.ftiles = a.n / kBF;
    a.nblocks = ((a.rows + kBT - 1) / kBT) * a.ftiles;
    if (a.nblocks == 0) return hipSuccess;
    if (a.dtype == T2H_F16) return gemm_typed<_Float16>(a, s);
    return gemm_typed<__bf16>(a, s);
}

}  // namespace t2h
