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
// Tiling: a block of 4 waves computes 256 features x 256 tokens (2 x 2 waves
// of 128 x 128: 16 MFMA tiles and 256 accumulators per lane, one wave per
// SIMD). K advances in steps of 64 through two 64 KB LDS stages filled by
// direct-to-LDS loads (global_load_lds_dwordx4: a wave's 64 lanes fill one
// contiguous KB); the 16-byte k chunks of each tile row are XOR-swizzled so
// that the fragment reads are conflict-free. The next stage's loads are in
// flight while the current stage's MFMAs run, and each substep's fragments
// are read while the previous substep's MFMAs run. Tile numbers are dealt
// to the 8 XCDs in contiguous ranges and walked in groups of a few token
// tiles, feature tile by feature tile, so the blocks resident on one XCD
// share a few weight and token slabs in its L2.
//
// Reference: GpuLinear.enqueue_gemm (gpu/linear.mojo:535-560, c[m, co] =
// a[m, ci] @ W^T), the MLP's lin0 + gelu_tanh_bias (gpu/linear.mojo:662-684,
// 776-809).
#include "t2h_device.h"
#include "t2h_internal.h"
#include "t2h_act.h"
#include "t2h_rope.h"

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
#ifndef T2H_GEMM_STAGES
#define T2H_GEMM_STAGES 2
#endif
#ifndef T2H_GEMM_DMAI
#define T2H_GEMM_DMAI 1
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
constexpr int kStages = T2H_GEMM_STAGES;  // LDS stages; loads run up to kStages stages ahead
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
static_assert(kStages >= 2 && kStages * kStageBytes <= 128 * 1024, "stages fit 128 KB of LDS");
static_assert((kStages - 1) * kLoads < 64, "vmcnt range");

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

// One k step (stage ks, in LDS buffer ks % kStages): kSub substeps of
// kFI x kTJ MFMAs. Substep s + 1's fragments are read while substep s's
// MFMAs run (the scheduling groups interleave 1 MFMA : 1 LDS read, then the
// remaining MFMAs). In the last substep, when NEXT: wait for stage ks + 1's
// loads (PEND later stages may still be in flight), the barrier that
// publishes them (after it every wave has finished reading stage ks), stage
// ks + kStages's loads into stage ks's buffer when ISSUE, and stage ks + 1's
// first fragments interleaved with the last MFMAs.
template <typename T, bool NEXT, bool ISSUE, int PEND>
__device__ __forceinline__ void stage_body(f32x16 (&acc)[kFI][kTJ], typename Mfma<T>::v8 (&af)[2][kFI],
                                           typename Mfma<T>::v8 (&bf)[2][kTJ], const StageCtx& cx, int ks) {
    const int buf = ks % kStages;
    const uint8_t* st = cx.lds + buf * kStageBytes;
#pragma unroll
    for (int s = 0; s < kSub; ++s) {
        const int c = s & 1, n = c ^ 1;
        const bool last = s + 1 == kSub;
        if (!last) {
            read_frags<T>(af[n], bf[n], st, cx.fa, cx.fb, cx.slot ^ (32 * (s + 1)));
        } else if (NEXT) {
            wait_vm<PEND * kLoads>();
            __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            if (ISSUE) issue_stage(cx.wbase, cx.xbase, cx.src, ks + kStages, cx.lds + buf * kStageBytes, cx.wave);
            read_frags<T>(af[n], bf[n], cx.lds + ((ks + 1) % kStages) * kStageBytes, cx.fa, cx.fb, cx.slot);
        }
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) acc[fi][tj] = Mfma<T>::run(af[c][fi], bf[c][tj], acc[fi][tj]);
        if (last && NEXT && ISSUE && T2H_GEMM_DMAI) {
            // the next stage's loads (kLoads per wave) go out between this
            // substep's first MFMAs, its first fragments between the rest
            // (the LDS reads stay behind the loads' m0 writes)
            constexpr int kG = kFI + kTJ;
            static_assert(kLoads % kG == 0 && kFI * kTJ >= 2 * kG, "groups");
#pragma unroll
            for (int g = 0; g < kG; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // MFMA
                __builtin_amdgcn_sched_group_barrier(0x010, kLoads / kG, 0);    // VMEM (to LDS)
            }
#pragma unroll
            for (int g = 0; g < kG; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);              // LDS read
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // MFMA
            }
            __builtin_amdgcn_sched_group_barrier(0x008, kFI * kTJ - 2 * kG, 0);
        } else if (!last || NEXT) {
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

// wait_vm<n * kLoads> for a small runtime stage count n
__device__ __forceinline__ void wait_stages(int n) {
    switch (n) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<kLoads>(); break;
        case 2: wait_vm<(kStages > 2 ? 2 : 1) * kLoads>(); break;
        default: wait_vm<(kStages > 3 ? 3 : 1) * kLoads>(); break;
    }
}

template <int ACT>
__device__ __forceinline__ float epi_f(float acc, float b) {
    const float v = bias_add(acc, b);
    if constexpr (ACT < 0) return v;
    else return act_f<ACT>(v);
}

#ifndef T2H_GEMM_TG
#define T2H_GEMM_TG 4
#endif
constexpr int kTokGroup = T2H_GEMM_TG;   // token tiles per group (0: token-tile-major order)

// Block tile of a launch: token tile t0 and feature tile n0 of block b. The
// XCD deal gives each XCD a contiguous range of tile numbers; within groups
// of kTokGroup token tiles the numbers walk feature tile by feature tile, so
// the blocks resident on an XCD at once share a few weight slabs and a few
// token slabs in its L2 (a bijection of [0, nblocks)).
struct TileOf {
    int64_t t0, n0;
    __device__ __forceinline__ bool init(const GemmArgs& a) {
        const int64_t b = block_linear();
        if (b >= a.nblocks) return false;
        const int64_t u = xcd_tile(b, a.nblocks);
        int64_t tt, ft;
        if constexpr (kTokGroup > 0) {
            const int64_t ntok = a.nblocks / a.ftiles;
            const int64_t gsz = (int64_t)kTokGroup * a.ftiles;
            const int64_t g = u / gsz, off = u - g * gsz;
            const int64_t rem = ntok - g * kTokGroup;
            const int64_t tg = rem < kTokGroup ? rem : kTokGroup;
            tt = g * kTokGroup + off % tg;
            ft = off / tg;
        } else {
            tt = u / a.ftiles;
            ft = u - tt * a.ftiles;
        }
        t0 = tt * kBT;
        n0 = ft * kBF;
        return true;
    }
};

// Residual rows of a 16-bit gated-residual tile into LDS: 32 rows per wave
// from `row0` (row r at r * 512 bytes, chunk c at slot c ^ (r % 32), the
// epilogue's staging layout), 2 rows per direct-to-LDS load: lane l fills
// slot l % 32 of row 2 it + l / 32. Rows past the last token read the last.
__device__ __forceinline__ void res_rows(const GemmArgs& a, int64_t t0, int64_t n0, uint8_t* lds, int row0, int wave,
                                         int lane) {
    const uint8_t* rb = static_cast<const uint8_t*>(a.res);
    const int64_t last = a.rows - 1;
    const int fr = lane & 31, h = lane >> 5;
#pragma unroll
    for (int it = 0; it < 16; ++it) {
        const int r = row0 + wave * 32 + it * 2 + h;
        const int64_t t = t0 + r < last ? t0 + r : last;
        const int c = fr ^ (r & 31);
        __builtin_amdgcn_global_load_lds(rb + (t * a.ldo + n0 + c * 8) * 2,
                                         lds + (row0 + wave * 32 + it * 2) * (kBF * 2), 16, 0, 0);
    }
}

// The block's accumulators acc[t0.., n0..] over all of k. On return every
// wave has finished reading the LDS stages (a barrier follows the last one),
// so the caller may reuse the LDS. RES_PRE: the last stage's MFMAs also
// cover the residual rows of the stage buffer it leaves free (rows
// [128 * (ksteps % 2), +128) of a 16-bit gated-residual tile).
template <typename T, bool RES_PRE = false>
__device__ __forceinline__ void gemm_mainloop(const GemmArgs& a, int64_t t0, int64_t n0, uint8_t* lds,
                                              f32x16 (&acc)[kFI][kTJ]) {
    using V8 = typename Mfma<T>::v8;
    static_assert(sizeof(T) == 2, "16-bit operands");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wf = wave & 1;
    const int wt = wave >> 1;
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

    // fragment slots: row lane % 32 of each MFMA tile, k chunk 2s + lane / 32;
    // (2s | h) ^ swz = (h ^ swz) ^ 2s, so substep s's slot is slot ^ 32s
    const int fr = lane & 31;
    const int h = lane >> 5;
    const int slot = (h ^ swz(fr)) * 16;
    const int fa = (wf * kWF + fr) * kRowBytes;             // row fr of the weight tile
    const int fb = kChunksA * 16 + (wt * kWT + fr) * kRowBytes;

    const int ksteps = a.k / kBK;
    // kStages LDS stages. The prologue issues the first kStages steps. At the
    // barrier in stage ks's last substep (stage ks + 1 has landed; up to
    // kStages - 2 later stages are in flight), every wave has finished reading
    // stage ks, so stage ks + kStages's loads go into stage ks's buffer, and
    // stage ks + 1's first fragments are read while stage ks's last MFMAs run.
    const int pro = ksteps < kStages ? ksteps : kStages;
#pragma unroll
    for (int st = 0; st < kStages; ++st)
        if (st < pro) issue_stage(wbase, xbase, src, st, lds + st * kStageBytes, wave);
    wait_stages(pro - 1);
    __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();

    V8 af[2][kFI], bf[2][kTJ];
    read_frags<T>(af[0], bf[0], lds, fa, fb, slot);
    __builtin_amdgcn_sched_barrier(0);
    // branch-free steady state, then the tail (no further loads; fewer
    // stages in flight), then the last stage (no next stage)
    const StageCtx cx{wbase, xbase, src, lds, fa, fb, slot, wave};
    int ks = 0;
    for (; ks + kStages < ksteps; ++ks) stage_body<T, true, true, kStages - 2>(acc, af, bf, cx, ks);
    // the last r = ksteps - ks <= kStages stages, straight-line: stage i of
    // the tail has r - 2 - i stages in flight after its next one
    static_assert(kStages <= 4, "tail cases");
    const int r = ksteps - ks;
    if (kStages > 3 && r >= 4) stage_body<T, true, false, (kStages > 3 ? 2 : 0)>(acc, af, bf, cx, ks++);
    if (kStages > 2 && r >= 3) stage_body<T, true, false, (kStages > 2 ? 1 : 0)>(acc, af, bf, cx, ks++);
    if (r >= 2) stage_body<T, true, false, 0>(acc, af, bf, cx, ks++);
    if constexpr (RES_PRE) {
        // stage ks + 1's buffer: no load targets it any more and every wave
        // finished reading it before the barrier of stage ks - 1
        static_assert(kStages == 2 && kStageBytes == 128 * kBF * 2, "a free stage holds 128 residual rows");
        res_rows(a, t0, n0, lds, ((ks + 1) % kStages) * 128, wave, lane);
    }
    stage_body<T, false, false, 0>(acc, af, bf, cx, ks);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();                // every wave is done reading the stages
}

__device__ __forceinline__ void zero_acc(f32x16 (&acc)[kFI][kTJ]) {
#pragma unroll
    for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
        for (int tj = 0; tj < kTJ; ++tj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fi][tj][r] = 0.0f;
}

// ---- linear: out = act(acc + bias) ------------------------------------------
// The lane holds token wt*kWT + tj*32 + fr of each token tile and features
// wf*kWF + fi*32 + 8q + 4h + 0..3. bias + activation are applied in f32 on
// the accumulators (one rounding to the output type). 16-bit outputs are
// staged in LDS as 256 token rows of 512 bytes (16-byte chunk c of row r at
// c ^ (r % 32): conflict-free both ways) and leave as whole rows, 16
// contiguous bytes per lane; f32 outputs go out directly.
template <typename T, typename O, int ACT>
__global__ __launch_bounds__(kGemmThreads, T2H_GEMM_OCC) void gemm_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];
    TileOf tile;
    if (!tile.init(a)) return;
    const int64_t t0 = tile.t0, n0 = tile.n0;
    f32x16 acc[kFI][kTJ];
    zero_acc(acc);
    gemm_mainloop<T>(a, t0, n0, lds, acc);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wf = wave & 1, wt = wave >> 1;
    const int fr = lane & 31, h = lane >> 5;
    O* __restrict__ out = static_cast<O*>(a.out);
    auto bias4 = [&](int fi, int q, float* bq) {
        if (a.bias != nullptr) {
            load_params<4>(a.bias + n0 + wf * kWF + fi * 32 + q * 8 + h * 4, bq);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) bq[i] = 0.0f;
        }
    };
    if constexpr (sizeof(O) == 2) {
        static_assert(kBT * kBF * 2 <= kStages * kStageBytes, "C tile fits the stage buffers");
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
            float bv[4][4];
#pragma unroll
            for (int q = 0; q < 4; ++q) bias4(fi, q, bv[q]);
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int r = wt * kWT + tj * 32 + fr;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int c = (wf * kWF + fi * 32 + q * 8) / 8;
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = epi_f<ACT>(acc[fi][tj][q * 4 + i], bv[q][i]);
                    u32x2 w;
                    w.x = Word<O>::pack(v);
                    w.y = Word<O>::pack(v + 2);
                    *reinterpret_cast<u32x2*>(lds + r * (kBF * 2) + ((c ^ (r & 31)) * 16) + h * 8) = w;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        constexpr int kRowsPerWave = kBT / 4;
#pragma unroll 4
        for (int it = 0; it < kRowsPerWave / 2; ++it) {
            const int r = wave * kRowsPerWave + it * 2 + h;
            const int c = fr;
            const int64_t t = t0 + r;
            const u32x4 w = *reinterpret_cast<const u32x4*>(lds + r * (kBF * 2) + ((c ^ (r & 31)) * 16));
            if (t < a.rows) *reinterpret_cast<u32x4*>(out + t * a.ldo + n0 + c * 8) = w;
        }
    } else {
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
            float bv[4][4];
#pragma unroll
            for (int q = 0; q < 4; ++q) bias4(fi, q, bv[q]);
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int64_t t = t0 + wt * kWT + tj * 32 + fr;
                if (t >= a.rows) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t n = n0 + wf * kWF + fi * 32 + q * 8 + h * 4;
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = epi_f<ACT>(acc[fi][tj][q * 4 + i], bv[q][i]);
                    store_elems<O, 4>(out + t * a.ldo + n, v);
                }
            }
        }
    }
}

// ---- linear + gated residual: out = res + fl(fl(acc + bias) * gate[b(t)]) ----
// The residual join of the block (x += (h + bias) * gate, or x += h + bias)
// in the store of the GEMM that makes h, so h never reaches memory; the
// rounding sequence is the gated-residual kernel's, with h = the f32 sums.
// 16-bit outputs: the residual tile is copied into the freed LDS stages with
// direct-to-LDS loads (each lane fetches the chunk that the staging swizzle
// puts at its slot; the half that lands in the stage buffer the last k step
// leaves free is requested before that step's MFMAs), each lane updates its
// values there in place, and whole rows leave as 16-byte stores. f32 outputs
// read and write the residual directly. out may alias res (every element is
// read before it is written, by the same thread).
template <typename T, typename O>
__global__ __launch_bounds__(kGemmThreads, T2H_GEMM_OCC) void gemm_res_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];
    TileOf tile;
    if (!tile.init(a)) return;
    const int64_t t0 = tile.t0, n0 = tile.n0;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wf = wave & 1, wt = wave >> 1;
    const int fr = lane & 31, h = lane >> 5;
    const BatchMap bm{a.batch.offsets, a.batch.rows_per_batch, a.batch.nbatch};
    const O* __restrict__ res = static_cast<const O*>(a.res);
    O* __restrict__ out = static_cast<O*>(a.out);
    const int64_t last = a.rows - 1;
    // gate row of the tile when all its rows share one batch (block-uniform),
    // else -1: each token looks up its own
    f32x16 acc[kFI][kTJ];
    zero_acc(acc);
    gemm_mainloop<T, sizeof(O) == 2>(a, t0, n0, lds, acc);
    int64_t tile_b = 0;
    if (a.gate != nullptr) {
        const int64_t tl = t0 + kBT - 1 < last ? t0 + kBT - 1 : last;
        const int32_t b0 = bm.batch_of(t0 < last ? t0 : last);
        tile_b = bm.batch_of(tl) == b0 ? b0 : -1;
    }
    // bias and gate of feature group fi (4 runs of 4 features per lane)
    auto params = [&](int fi, float (&bv)[4][4], float (&gv)[4][4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int64_t n = n0 + wf * kWF + fi * 32 + q * 8 + h * 4;
            if (a.bias != nullptr) load_params<4>(a.bias + n, bv[q]);
            if (a.gate != nullptr && tile_b >= 0) load_params<4>(a.gate + tile_b * a.gate_stride + n, gv[q]);
        }
    };
    // u = res + fl(fl(acc + bias) * gate) for token tile tj, group (fi, q)
    auto join4 = [&](int fi, int tj, int q, const float* bq, const float* gq, const float* rv, float* u) {
        float g[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) g[i] = gq[i];
        if (a.gate != nullptr && tile_b < 0) {
            const int64_t t = t0 + wt * kWT + tj * 32 + fr;
            load_params<4>(a.gate + bm.batch_of(t < last ? t : last) * a.gate_stride + n0 + wf * kWF + fi * 32 +
                               q * 8 + h * 4, g);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = a.bias != nullptr ? add_rn(acc[fi][tj][q * 4 + i], bq[i]) : acc[fi][tj][q * 4 + i];
            if (a.gate != nullptr) v = mul_rn(v, g[i]);
            u[i] = add_rn(rv[i], v);
        }
    };
    if constexpr (sizeof(O) == 2) {
        static_assert(kBT * kBF * 2 <= kStages * kStageBytes, "C tile fits the stage buffers");
        constexpr int kRowsPerWave = kBT / 4;
        // residual rows -> LDS: the last stage left rows [128 * (ksteps % 2),
        // +128) loading; now the other half, and every bias and gate value
        // of the lane, all in flight together
        res_rows(a, t0, n0, lds, (1 - (a.k / kBK) % 2) * 128, wave, lane);
        float bv[kFI][4][4], gv[kFI][4][4];
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) params(fi, bv[fi], gv[fi]);
        wait_vm<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int r = wt * kWT + tj * 32 + fr;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int c = (wf * kWF + fi * 32 + q * 8) / 8;
                    u32x2* p = reinterpret_cast<u32x2*>(lds + r * (kBF * 2) + ((c ^ (r & 31)) * 16) + h * 8);
                    const u32x2 w0 = *p;
                    float rv[4], u[4];
                    Word<O>::unpack(w0.x, rv);
                    Word<O>::unpack(w0.y, rv + 2);
                    join4(fi, tj, q, bv[fi][q], gv[fi][q], rv, u);
                    u32x2 w;
                    w.x = Word<O>::pack(u);
                    w.y = Word<O>::pack(u + 2);
                    *p = w;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
#pragma unroll 4
        for (int it = 0; it < kRowsPerWave / 2; ++it) {
            const int r = wave * kRowsPerWave + it * 2 + h;
            const int c = fr;
            const int64_t t = t0 + r;
            const u32x4 w = *reinterpret_cast<const u32x4*>(lds + r * (kBF * 2) + ((c ^ (r & 31)) * 16));
            if (t < a.rows) *reinterpret_cast<u32x4*>(out + t * a.ldo + n0 + c * 8) = w;
        }
    } else {
        // per feature group: its residual values and parameters are all
        // loaded before its first store (loads and stores share vmcnt on
        // gfx9: a load consumed while a store is pending waits for the store)
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
            float bv[4][4], gv[4][4];
            params(fi, bv, gv);
            float rv[kTJ][4][4];
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int64_t t = t0 + wt * kWT + tj * 32 + fr;
                const int64_t tc = t < a.rows ? t : last;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    load_elems<O, 4>(res + tc * a.ldo + n0 + wf * kWF + fi * 32 + q * 8 + h * 4, rv[tj][q]);
            }
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int64_t t = t0 + wt * kWT + tj * 32 + fr;
                if (t >= a.rows) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float u[4];
                    join4(fi, tj, q, bv[q], gv[q], rv[tj][q], u);
                    store_elems<O, 4>(out + t * a.ldo + n0 + wf * kWF + fi * 32 + q * 8 + h * 4, u);
                }
            }
        }
    }
}

// ---- qkv linear + attention epilogue + head-major pack ----------------------
// The qkv GEMM's output [rows, 3, H, 128] never reaches memory. A wave's 128
// features are one head (q, k or v: head hg = n / 128, tensor hg / H, head
// hg % H) for 128 tokens, and each token's head lives in two lanes (l and
// l ^ 32, 64 values each). Per token, in the order of the separate kernels
// (bias_rms_rope_qkv, pack_q_z, pack_kv_z): + bias; q/k: RMS over the head,
// x * rsqrt(sum x^2) * (gamma * sqrt(D)); q/k: RoPE on the in-lane pairs
// (2p, 2p + 1) with cos/sin from the phase table or from the token's
// position; q: * 1/sqrt(D); tokens >= rows: 0. The head then goes through
// the wave's own 16 KB of LDS, 64 tokens at a time, as 256-byte token rows
// and leaves as 16-byte vectors: whole token rows (qh [H, mp, D], k [H, lp,
// D], vh [H, lp, D]) or, for the transposed k [H, D, lp], 8 tokens of one
// feature gathered from 8 rows. Tiles past the last token row skip the GEMM
// and write the pads.
constexpr int kHead = 128;
static_assert(kTJ == 2 || kTJ == 4, "copy_col cases");

// Slot of a 16-byte chunk in a staged 256-byte token row: chunk c of row r
// at c ^ stage_swz(r). Over 32 consecutive rows (one row-major write) every
// slot appears twice; over rows 8g + j, g = 0..7 (one transposed gather)
// the slots are distinct; a row's 16 chunks are a permutation.
__device__ __forceinline__ int stage_swz(int r) { return ((r >> 3) ^ ((r & 7) << 1)) & 15; }

template <int TJ>
__device__ __forceinline__ void copy_col(const f32x16 (&acc)[kFI][kTJ], float (&col)[kFI][16]) {
#pragma unroll
    for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
        for (int r = 0; r < 16; ++r) col[fi][r] = acc[fi][TJ][r];
}

template <typename T, bool KT>
__global__ __launch_bounds__(kGemmThreads, T2H_GEMM_OCC) void qkv_pack_kernel(GemmArgs g, PackArgs p, RopeSlots tab) {
    // One LDS array: the GEMM's stages, then the epilogue's staging (4 waves
    // x 16 KB: 64 token rows of 256 bytes) and the tile's parameters at 64 KB.
    // (A separate parameter array that took the kernel past 128 KB of LDS
    // measured 20 % slower on MI355X.)
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];
    static_assert(kWF == kHead && kWT % 64 == 0 && 4 * 64 * 256 + 2 * 2 * kHead * 4 <= kStages * kStageBytes,
                  "staging layout");
    TileOf tile;
    if (!tile.init(g)) return;
    const int64_t t0 = tile.t0, n0 = tile.n0;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wf = wave & 1, wt = wave >> 1;
    const int fr = lane & 31, h = lane >> 5;
    const int hg = (int)((n0 + wf * kWF) / kHead);
    const int which = hg / p.heads;          // 0 q, 1 k, 2 v (the block's two heads share it)
    const int z = hg - which * p.heads;
    const float* __restrict__ bias = which == 0 ? p.bias_q : which == 1 ? p.bias_k : p.bias_v;
    const float* __restrict__ gamma = which == 0 ? p.gamma_q : which == 1 ? p.gamma_k : nullptr;

    // the tile's bias and gamma * sqrt(D) (one value of each per thread) are
    // requested before the GEMM and land in LDS after it
    static_assert(kGemmThreads == 2 * kHead, "one parameter per thread and head");
    const int ph_ = threadIdx.x / kHead, pd_ = threadIdx.x % kHead;
    const int pz_ = (int)((n0 + ph_ * kWF) / kHead) - which * p.heads;
    const float pbias = bias != nullptr ? bias[pz_ * kHead + pd_] : 0.0f;
    const float pgam = gamma != nullptr ? gamma[pz_ * kHead + pd_] : 0.0f;
    f32x16 acc[kFI][kTJ];
    zero_acc(acc);
    if (t0 < g.rows) gemm_mainloop<T>(g, t0, n0, lds, acc);   // block-uniform (ends with a barrier)
    float* prm = reinterpret_cast<float*>(lds + 4 * 64 * 256);   // [head][bias, gamma*sqrt(D)][128]
    prm[(ph_ * 2 + 0) * kHead + pd_] = pbias;
    prm[(ph_ * 2 + 1) * kHead + pd_] = pgam * p.rms_scale;
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();

    const bool rope = p.use_rope && which < 2 && g.rows > 0;
    const int64_t extent = which == 0 ? p.mp : p.lp;
    T* __restrict__ out = static_cast<T*>(which == 0 ? p.qh : which == 1 ? p.k_out : p.vh);
    const bool trans = KT && which == 1;
    uint8_t* region = lds + wave * (64 * 256);
    const float* pb = prm + (wf * 2 + 0) * kHead;
    const float* pg = prm + (wf * 2 + 1) * kHead;

#pragma unroll 1
    for (int half = 0; half < kTJ / 2; ++half) {
#pragma unroll 1
        for (int jj = 0; jj < 2; ++jj) {
            const int tj = half * 2 + jj;
            // this token tile's accumulators (static register indices per case)
            float col[kFI][16];
            switch (tj) {
                case 0: copy_col<0>(acc, col); break;
                case 1: copy_col<1>(acc, col); break;
                case 2: copy_col<(kTJ > 2 ? 2 : 0)>(acc, col); break;
                default: copy_col<(kTJ > 2 ? 3 : 1)>(acc, col); break;
            }
            const int tl = jj * 32 + fr;                      // staged row (token within the half)
            const int64_t t = t0 + wt * kWT + tj * 32 + fr;
            const int64_t tc = t < g.rows ? t : g.rows - 1;   // clamped for position reads
            const bool live = t < g.rows;
            // feature of col[fi][4q + i]: d = fi*32 + 8q + 4h + i
            // the token's cos/sin (table path) are requested first and arrive
            // while the bias and the sum of squares are computed
            float cs[kFI][4][4];
            const bool table = rope && p.phases != nullptr;
            if (table) {
                const float* row = p.phases + (tc % p.phase_rows) * kHead;
#pragma unroll
                for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
                    for (int q = 0; q < 4; ++q) load_params<4>(row + fi * 32 + q * 8 + h * 4, cs[fi][q]);
            }
            if (bias != nullptr) {
#pragma unroll
                for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 b4 = *reinterpret_cast<const float4*>(pb + fi * 32 + q * 8 + h * 4);
                        col[fi][q * 4 + 0] = add_rn(col[fi][q * 4 + 0], b4.x);
                        col[fi][q * 4 + 1] = add_rn(col[fi][q * 4 + 1], b4.y);
                        col[fi][q * 4 + 2] = add_rn(col[fi][q * 4 + 2], b4.z);
                        col[fi][q * 4 + 3] = add_rn(col[fi][q * 4 + 3], b4.w);
                    }
            }
            // the head's sum of squares: 64 values here, 64 in lane ^ 32
            float rn = 1.0f;
            if (gamma != nullptr) {
                float ss = 0.0f;
#pragma unroll
                for (int fi = 0; fi < kFI; ++fi) ss += sum_sq<16>(col[fi]);
                ss += __shfl_xor(ss, 32);
                rn = ss < 1e-24f ? 1e12f : __builtin_amdgcn_rsqf(ss);
            }
            float pos[T2H_MAX_POS_DIM];
            if (rope && !table) {
                const PosSource src{p.coords, p.coord_cols, p.grid_res, p.pos_dim};
                src.get(tc, pos);
            }
#pragma unroll
            for (int fi = 0; fi < kFI; ++fi) {
                float* v = col[fi];
                if (gamma != nullptr) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 g4 = *reinterpret_cast<const float4*>(pg + fi * 32 + q * 8 + h * 4);
                        v[q * 4 + 0] = (v[q * 4 + 0] * rn) * g4.x;
                        v[q * 4 + 1] = (v[q * 4 + 1] * rn) * g4.y;
                        v[q * 4 + 2] = (v[q * 4 + 2] * rn) * g4.z;
                        v[q * 4 + 3] = (v[q * 4 + 3] * rn) * g4.w;
                    }
                }
                if (rope) {
                    if (table) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            rotate_pair(v[q * 4 + 0], v[q * 4 + 1], cs[fi][q][0], cs[fi][q][1]);
                            rotate_pair(v[q * 4 + 2], v[q * 4 + 3], cs[fi][q][2], cs[fi][q][3]);
                        }
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q)
#pragma unroll
                            for (int j = 0; j < 2; ++j) {
                                const int sl = (fi * 32 + q * 8 + h * 4) / 2 + j;
                                float c, sn;
                                slot_phase(pos, tab.axis[sl], tab.freq[sl], c, sn);
                                rotate_pair(v[q * 4 + 2 * j], v[q * 4 + 2 * j + 1], c, sn);
                            }
                    }
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float x = which == 0 ? mul_rn(v[r], p.q_scale) : v[r];
                    v[r] = live ? x : 0.0f;
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int c = fi * 4 + q;                  // 16-byte chunk of the 256-byte token row
                    u32x2 w;
                    w.x = Word<T>::pack(&v[q * 4]);
                    w.y = Word<T>::pack(&v[q * 4 + 2]);
                    *reinterpret_cast<u32x2*>(region + tl * 256 + ((c ^ stage_swz(tl)) * 16) + h * 8) = w;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);      // the wave's LDS writes are done (its region is private)
        const int64_t tw = t0 + wt * kWT + half * 64;   // first token of the staged rows
        if (!trans) {
            // token rows: 16 lanes per 256-byte row, 4 rows per instruction
#pragma unroll 4
            for (int it = 0; it < 64 / 4; ++it) {
                const int row = it * 4 + (lane >> 4);
                const int c = lane & 15;
                const u32x4 w = *reinterpret_cast<const u32x4*>(region + row * 256 + ((c ^ stage_swz(row)) * 16));
                const int64_t t = tw + row;
                if (t < extent) *reinterpret_cast<u32x4*>(out + ((int64_t)z * extent + t) * kHead + c * 8) = w;
            }
        } else {
            // feature rows of the transposed k: lane (d, g) gathers feature d
            // of tokens 8g .. 8g + 7 (eight 2-byte reads, one per token row)
#pragma unroll 2
            for (int it = 0; it < kHead / 8; ++it) {
                const int d = it * 8 + (lane >> 3);
                const int gg = lane & 7;
                const int off = (d & 7) * 2;
                uint32_t wv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r0 = gg * 8 + 2 * j, r1 = r0 + 1;
                    const uint32_t lo = *reinterpret_cast<const uint16_t*>(
                        region + r0 * 256 + (((d >> 3) ^ stage_swz(r0)) * 16) + off);
                    const uint32_t hi = *reinterpret_cast<const uint16_t*>(
                        region + r1 * 256 + (((d >> 3) ^ stage_swz(r1)) * 16) + off);
                    wv[j] = lo | (hi << 16);
                }
                const int64_t t = tw + gg * 8;
                if (t < extent) {
                    u32x4 w;
                    w.x = wv[0];
                    w.y = wv[1];
                    w.z = wv[2];
                    w.w = wv[3];
                    *reinterpret_cast<u32x4*>(out + ((int64_t)z * kHead + d) * p.lp + t) = w;
                }
            }
        }
        // the next half overwrites the staged rows: every lane's reads are done
        __builtin_amdgcn_s_waitcnt(0xC07F);
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

template <typename T>
hipError_t gemm_res_typed(const GemmArgs& a, hipStream_t s) {
    const dim3 g = grid_1d(a.nblocks), blk(kGemmThreads);
    if (a.out_dtype == T2H_F32) hipLaunchKernelGGL((gemm_res_kernel<T, float>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((gemm_res_kernel<T, T>), g, blk, 0, s, a);
    return hipGetLastError();
}

template <typename T>
hipError_t qkv_typed(const GemmArgs& g, const PackArgs& p, const RopeSlots& tab, hipStream_t s) {
    const dim3 grid = grid_1d(g.nblocks), blk(kGemmThreads);
    if (p.k_transposed) hipLaunchKernelGGL((qkv_pack_kernel<T, true>), grid, blk, 0, s, g, p, tab);
    else hipLaunchKernelGGL((qkv_pack_kernel<T, false>), grid, blk, 0, s, g, p, tab);
    return hipGetLastError();
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

hipError_t launch_gemm_residual(GemmArgs a, hipStream_t s) {
    a.ftiles = a.n / kBF;
    a.nblocks = ((a.rows + kBT - 1) / kBT) * a.ftiles;
    if (a.nblocks == 0) return hipSuccess;
    if (a.dtype == T2H_F16) return gemm_res_typed<_Float16>(a, s);
    return gemm_res_typed<__bf16>(a, s);
}

int32_t gemm_head_dim() { return kHead; }

hipError_t launch_qkv_pack(GemmArgs g, const PackArgs& p, const RopeSlots& tab, hipStream_t s) {
    // token tiles cover the pad rows of the outputs too (they are written as 0)
    int64_t span = g.rows;
    if (p.mp > span) span = p.mp;
    if (p.lp > span) span = p.lp;
    g.ftiles = g.n / kBF;
    g.nblocks = ((span + kBT - 1) / kBT) * g.ftiles;
    if (g.nblocks == 0) return hipSuccess;
    if (g.dtype == T2H_F16) return qkv_typed<_Float16>(g, p, tab, s);
    return qkv_typed<__bf16>(g, p, tab, s);
}

}  // namespace t2h
