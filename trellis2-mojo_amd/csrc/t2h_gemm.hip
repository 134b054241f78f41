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

#ifndef T2H_GEMM_BT
#define T2H_GEMM_BT 256
#endif
#ifndef T2H_GEMM_BK
#define T2H_GEMM_BK 64
#endif
#ifndef T2H_GEMM_OCC
#define T2H_GEMM_OCC 1
#endif

constexpr int kGemmThreads = 256;
constexpr int kBF = 256;                  // features per block
constexpr int kBT = T2H_GEMM_BT;          // tokens per block
constexpr int kBK = T2H_GEMM_BK;          // k per stage
constexpr int kCpr = kBK / 8;             // 16-byte chunks per tile row
constexpr int kSub = kBK / 16;            // MFMA k substeps per stage
constexpr int kStages = 2;               // LDS stages (double buffer)
constexpr int kWF = kBF / 2;              // features per wave
constexpr int kWT = kBT / 2;              // tokens per wave
constexpr int kFI = kWF / 32;             // MFMA tiles along features
constexpr int kTJ = kWT / 32;             // MFMA tiles along tokens
constexpr int kRowBytes = kBK * 2;
constexpr int kChunksA = kBF * kCpr;      // 16-byte chunks of the weight tile per stage
constexpr int kChunksB = kBT * kCpr;      // ... of the token tile
constexpr int kStageBytes = (kChunksA + kChunksB) * 16;
constexpr int kLoadsA = kChunksA / 64 / 4;   // 64-lane loads per wave per stage
constexpr int kLoadsB = kChunksB / 64 / 4;
constexpr int kLoads = kLoadsA + kLoadsB;
static_assert(kCpr == 4 || kCpr == 8, "k step of 32 or 64");
static_assert(kLoads < 64, "vmcnt range");

// Tile u of nb, dealt so that XCD x (blocks b with b % 8 == x) takes the
// contiguous range of tiles [x*q + min(x, r), ...): a bijection of [0, nb).
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t nb) {
    const int64_t q = nb >> 3, r = nb & 7, x = b & 7, k = b >> 3;
    return x * q + (x < r ? x : r) + k;
}

// LDS layout of a tile row (kCpr 16-byte k chunks): chunk kc sits at slot
// kc ^ swz(row). The 16-byte fragment reads of 8 (or 16) consecutive rows at
// one k chunk then hit distinct bank groups of a 128 (or 256) byte LDS line.
// swz depends on row % 32 only, so a fragment read can take it from its row
// within the 32-row MFMA tile.
__device__ __forceinline__ int swz(int r) {
    if constexpr (kCpr == 4) return ((r >> 1) ^ (r >> 3)) & 3;
    else return ((r & 15) ^ ((r & 15) >> 3)) & 7;
}

// Wait until at most N of this wave's vector-memory operations are pending
// (vmcnt only; gfx9 encoding: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Issue one k step's loads of this wave into the LDS stage `st`: load i
// fills the 64 chunks [(i*4 + wave)*64, +64), one 16-byte chunk per lane.
// Byte addressing (both operand types are 2 bytes wide); src[] holds each
// load's byte offset from its tile base.
__device__ __forceinline__ void issue_stage(const uint8_t* wbase, const uint8_t* xbase, const int64_t* src, int ks,
                                            uint8_t* st, int wave) {
    const int64_t ko = (int64_t)ks * kBK * 2;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const uint8_t* g = (i < kLoadsA ? wbase : xbase) + src[i] + ko;
        __builtin_amdgcn_global_load_lds(g, st + (i * 4 + wave) * 1024, 16, 0, 0);
    }
}

// The wave's fragments of one k substep from LDS stage st: kFI weight
// fragments and kTJ token fragments, 16 bytes per lane each.
template <typename T, typename V8>
__device__ __forceinline__ void read_frags_impl(V8* af, V8* bf, const uint8_t* st, int fa, int fb, int so) {
#pragma unroll
    for (int fi = 0; fi < kFI; ++fi) af[fi] = *reinterpret_cast<const V8*>(st + fa + fi * 32 * kRowBytes + so);
#pragma unroll
    for (int tj = 0; tj < kTJ; ++tj) bf[tj] = *reinterpret_cast<const V8*>(st + fb + tj * 32 * kRowBytes + so);
}
template <typename T>
__device__ __forceinline__ void read_frags(typename Mfma<T>::v8* af, typename Mfma<T>::v8* bf, const uint8_t* st,
                                           int fa, int fb, int so) {
    read_frags_impl<T, typename Mfma<T>::v8>(af, bf, st, fa, fb, so);
}

struct StageCtx {
    const uint8_t* wbase;
    const uint8_t* xbase;
    const int64_t* src;
    uint8_t* lds;
    int fa, fb, slot, wave;
};

// One k step (stage ks, in LDS buffer ks & 1): kSub substeps of kFI x kTJ
// MFMAs. Substep s + 1's fragments are read while substep s's MFMAs run (the
// scheduling groups interleave 1 MFMA : 1 LDS read, then the remaining
// MFMAs). In the last substep, when NEXT: wait for stage ks + 1's loads, the
// barrier that publishes them (after it every wave has finished reading
// stage ks), stage ks + 2's loads into stage ks's buffer when ISSUE, and
// stage ks + 1's first fragments interleaved with the last MFMAs.
template <typename T, bool NEXT, bool ISSUE>
__device__ __forceinline__ void stage_body(f32x16 (&acc)[kFI][kTJ], typename Mfma<T>::v8 (&af)[2][kFI],
                                           typename Mfma<T>::v8 (&bf)[2][kTJ], const StageCtx& cx, int ks) {
    const uint8_t* st = cx.lds + (ks & 1) * kStageBytes;
#pragma unroll
    for (int s = 0; s < kSub; ++s) {
        const int c = s & 1, n = c ^ 1;
        const bool last = s + 1 == kSub;
        if (!last) {
            read_frags<T>(af[n], bf[n], st, cx.fa, cx.fb, cx.slot ^ (32 * (s + 1)));
        } else if (NEXT) {
            wait_vm<0>();
            __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            if (ISSUE) issue_stage(cx.wbase, cx.xbase, cx.src, ks + 2, cx.lds + (ks & 1) * kStageBytes, cx.wave);
            read_frags<T>(af[n], bf[n], cx.lds + ((ks + 1) & 1) * kStageBytes, cx.fa, cx.fb, cx.slot);
        }
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) acc[fi][tj] = Mfma<T>::run(af[c][fi], bf[c][tj], acc[fi][tj]);
        if (!last || NEXT) {
#pragma unroll
            for (int g = 0; g < kFI + kTJ; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
            }
            __builtin_amdgcn_sched_group_barrier(0x008, kFI * kTJ - (kFI + kTJ), 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int ACT>
__device__ __forceinline__ float epi_f(float acc, float b) {
    const float v = bias_add(acc, b);
    if constexpr (ACT < 0) return v;
    else return act_f<ACT>(v);
}

template <typename T, typename O, int ACT>
__global__ __launch_bounds__(kGemmThreads, T2H_GEMM_OCC) void gemm_kernel(GemmArgs a) {
    using V8 = typename Mfma<T>::v8;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];

    const int64_t b = block_linear();
    if (b >= a.nblocks) return;
    const int64_t u = xcd_tile(b, a.nblocks);
    const int64_t tt = u / a.ftiles;
    const int ft = (int)(u - tt * a.ftiles);
    const int64_t t0 = tt * kBT;
    const int64_t n0 = (int64_t)ft * kBF;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wf = wave & 1;
    const int wt = wave >> 1;

    static_assert(sizeof(T) == 2, "16-bit operands");
    const uint8_t* wbase = static_cast<const uint8_t*>(a.w) + n0 * (int64_t)a.k * 2;
    const uint8_t* xbase = static_cast<const uint8_t*>(a.x) + t0 * a.ldx * 2;
    const int64_t tlast = a.rows - 1 - t0;   // last valid token row of the tile

    // Loads straight into LDS: load i of wave w fills the 64 chunks
    // [(i*4 + w)*64, +64) of a stage (weight tile first, then token tile), one
    // 16-byte chunk per lane; each lane fetches the global chunk that the
    // swizzle puts at its slot. Pad tokens read the last row.
    int64_t src[kLoads];   // byte offsets
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int p = (i * 4 + wave) * 64 + lane;
        if (i < kLoadsA) {
            const int row = p / kCpr, kc = (p % kCpr) ^ swz(row);
            src[i] = ((int64_t)row * a.k + kc * 8) * 2;
        } else {
            const int q = p - kChunksA;
            const int row = q / kCpr, kc = (q % kCpr) ^ swz(row);
            const int64_t tr = row < tlast ? row : tlast;
            src[i] = (tr * a.ldx + kc * 8) * 2;
        }
    }

    f32x16 acc[kFI][kTJ];
#pragma unroll
    for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
        for (int tj = 0; tj < kTJ; ++tj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fi][tj][r] = 0.0f;

    // fragment slots: row lane % 32 of each MFMA tile, k chunk 2s + lane / 32;
    // (2s | h) ^ swz = (h ^ swz) ^ 2s, so substep s's slot is slot ^ 32s
    const int fr = lane & 31;
    const int h = lane >> 5;
    const int slot = (h ^ swz(fr)) * 16;
    const int fa = (wf * kWF + fr) * kRowBytes;             // row fr of the weight tile
    const int fb = kChunksA * 16 + (wt * kWT + fr) * kRowBytes;

    const int ksteps = a.k / kBK;
    // Two LDS stages. Stage ks + 1's loads are issued while stage ks is
    // computed; the barrier that publishes them sits in stage ks's last
    // substep, so stage ks + 1's first fragments are read while stage ks's
    // last MFMAs run. Right after that barrier every wave has finished
    // reading stage ks (its reads completed before the barrier), so stage
    // ks + 2's loads go into stage ks's buffer.
    issue_stage(wbase, xbase, src, 0, lds, wave);
    if (ksteps > 1) {
        issue_stage(wbase, xbase, src, 1, lds + kStageBytes, wave);
        wait_vm<kLoads>();
    } else {
        wait_vm<0>();
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();

    V8 af[2][kFI], bf[2][kTJ];
    read_frags<T>(af[0], bf[0], lds, fa, fb, slot);
    __builtin_amdgcn_sched_barrier(0);
    // branch-free steady state, then the last two stages (no further loads;
    // no next stage)
    const StageCtx cx{wbase, xbase, src, lds, fa, fb, slot, wave};
    int ks = 0;
    for (; ks + 2 < ksteps; ++ks) stage_body<T, true, true>(acc, af, bf, cx, ks);
    if (ks + 1 < ksteps) stage_body<T, true, false>(acc, af, bf, cx, ks++);
    stage_body<T, false, false>(acc, af, bf, cx, ks);

    // epilogue: lane holds token t of each token tile and features
    // n + 8q + 4(lane / 32) + 0..3 of each feature tile
    O* __restrict__ out = static_cast<O*>(a.out);
#pragma unroll
    for (int tj = 0; tj < kTJ; ++tj) {
        const int64_t t = t0 + wt * kWT + tj * 32 + fr;
        if (t >= a.rows) continue;
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t n = n0 + wf * kWF + fi * 32 + q * 8 + h * 4;
                float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (a.bias != nullptr) load_params<4>(a.bias + n, bv);
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = epi_f<ACT>(acc[fi][tj][q * 4 + i], bv[i]);
                store_elems<O, 4>(out + t * a.ldo + n, v);
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
