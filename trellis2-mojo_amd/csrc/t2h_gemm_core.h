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
// Tiling: a block computes 256 features x 256 tokens. K advances in steps of
// 64 through two 64 KB LDS stages; the 16-byte k chunks of each tile row are
// XOR-swizzled so that the fragment reads are conflict-free, and each
// substep's fragments are read while the previous substep's MFMAs run. Two
// layouts share this file (T2H_GEMM_WAVES, set by the translation unit):
// - 4 waves (2 x 2 of 128 x 128: 16 MFMA tiles, 256 accumulators per lane,
//   one wave per SIMD); the stages are filled by direct-to-LDS loads
//   (global_load_lds_dwordx4: a wave's 64 lanes fill one contiguous KB), the
//   next stage's in flight while the current one's MFMAs run. It is kept as
//   a build option (T2H_GEMM_WAVES / T2H_QKV_WAVES = 4).
// - 8 waves (2 x 4 of 128 x 64: 8 MFMA tiles, 128 accumulators, two waves
//   per SIMD); the next stage goes through registers: each wave writes it to
//   LDS a slice per substep and refills the slice's registers with the stage
//   after, and a wave raises its priority over its MFMAs. Every shipped
//   kernel uses it: linear and gated residual 2-5 % faster than the 4-wave
//   form, the fused qkv 10 %.
// Tile numbers are dealt to the 8 XCDs in contiguous ranges and walked in
// groups of a few token tiles, feature tile by feature tile, so the blocks
// resident on one XCD share a few weight and token slabs in its L2.
//
// Reference: GpuLinear.enqueue_gemm (gpu/linear.mojo:535-560, c[m, co] =
// a[m, ci] @ W^T), the MLP's lin0 + gelu_tanh_bias (gpu/linear.mojo:662-684,
// 776-809).
#pragma once
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

#ifndef T2H_GEMM_WAVES
#define T2H_GEMM_WAVES 4
#endif
constexpr int kWaves = T2H_GEMM_WAVES;     // 4 (one wave per SIMD) or 8 (two)
static_assert(kWaves == 4 || kWaves == 8, "wave layouts");
constexpr bool kRegStaged = kWaves == 8;   // stages through registers instead of direct-to-LDS loads
constexpr int kGemmThreads = 64 * kWaves;
constexpr int kBF = 256;                  // features per block
constexpr int kBT = T2H_GEMM_BT;          // tokens per block
constexpr int kBK = T2H_GEMM_BK;          // k per stage
constexpr int kCpr = kBK / 8;             // 16-byte chunks per tile row
constexpr int kSub = kBK / 16;            // MFMA k substeps per stage
constexpr int kStages = T2H_GEMM_STAGES;  // LDS stages; loads run up to kStages stages ahead
constexpr int kWF = kBF / 2;              // features per wave
constexpr int kWT = kBT / (kWaves / 2);   // tokens per wave
constexpr int kFI = kWF / 32;             // MFMA tiles along features
constexpr int kTJ = kWT / 32;             // MFMA tiles along tokens
constexpr int kRowBytes = kBK * 2;
constexpr int kChunksA = kBF * kCpr;      // 16-byte chunks of the weight tile per stage
constexpr int kChunksB = kBT * kCpr;      // ... of the token tile
constexpr int kStageBytes = (kChunksA + kChunksB) * 16;
constexpr int kLoadsA = kChunksA / 64 / kWaves;   // 64-lane loads per wave per stage
constexpr int kLoadsB = kChunksB / 64 / kWaves;
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
// fills the 64 chunks [(i*kWaves + wave)*64, +64), one 16-byte chunk per lane.
// Byte addressing (both operand types are 2 bytes wide); src[] holds each
// load's byte offset from its tile base.
__device__ __forceinline__ void issue_stage(const uint8_t* wbase, const uint8_t* xbase, const int64_t* src, int ks,
                                            uint8_t* st, int wave) {
    const int64_t ko = (int64_t)ks * kBK * 2;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const uint8_t* g = (i < kLoadsA ? wbase : xbase) + src[i] + ko;
        __builtin_amdgcn_global_load_lds(g, st + (i * kWaves + wave) * 1024, 16, 0, 0);
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

// Token tiles per group of the tile order (0: token-tile-major): 4, or 2 for
// K >= 4096, where a token tile's operand slab is 4 times as long (measured on
// MI355X: 2 is 0.7 % faster for K = 6144 and 1.5-2 % slower for K = 1536).
__host__ __device__ inline int tile_group(int k) { return k >= 4096 ? 2 : 4; }

// Block tile of a launch: token tile t0 and feature tile n0 of block b. The
// XCD deal gives each XCD a contiguous range of tile numbers; within groups
// of a.tgroup token tiles the numbers walk feature tile by feature tile, so
// the blocks resident on an XCD at once share a few weight slabs and a few
// token slabs in its L2 (a bijection of [0, nblocks)).
struct TileOf {
    int64_t t0, n0;
    __device__ __forceinline__ bool init(const GemmArgs& a) {
        const int64_t b = block_linear();
        if (b >= a.nblocks) return false;
        const int64_t u = xcd_tile(b, a.nblocks);
        int64_t tt, ft;
        if (a.tgroup > 0) {
            const int64_t ntok = a.nblocks / a.ftiles;
            const int64_t gsz = (int64_t)a.tgroup * a.ftiles;
            const int64_t g = u / gsz, off = u - g * gsz;
            const int64_t rem = ntok - g * a.tgroup;
            const int64_t tg = rem < a.tgroup ? rem : a.tgroup;
            tt = g * a.tgroup + off % tg;
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

// ---- register-staged stages (8 waves) ----
// During stage ks each wave writes stage ks + 1's chunks from VGPRs into the
// free buffer (ks + 1) % 2, a slice per substep (substeps 0 .. kSub - 2), and
// refills each slice's registers with stage ks + 2's chunks right after
// writing it. Chunk i of wave w is the 1 KB at (i*kWaves + w) KB of a stage,
// lane l's 16 bytes at l * 16.
__device__ __forceinline__ constexpr int rs_lo(int s) { return kLoads * s / (kSub - 1); }
__device__ __forceinline__ void rs_fetch(u32x4 (&r)[kLoads], const uint8_t* wbase, const uint8_t* xbase,
                                        const int64_t* src, int ks, int lo, int hi) {
    const int64_t ko = (int64_t)ks * kBK * 2;
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
        if (i >= lo && i < hi)
            r[i] = *reinterpret_cast<const u32x4*>((i < kLoadsA ? wbase : xbase) + src[i] + ko);
}
__device__ __forceinline__ void rs_write(const u32x4 (&r)[kLoads], uint8_t* st, int wave, int lane, int lo, int hi) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
        if (i >= lo && i < hi) *reinterpret_cast<u32x4*>(st + (i * kWaves + wave) * 1024 + lane * 16) = r[i];
}
// Scheduling of one substep's MFMAs: MFMA g carries a fragment read when
// g < NR, and an LDS write (plus, with LOAD, the refill load) when
// g >= MFMAs - NW.
template <int NR, int NW, bool LOAD>
__device__ __forceinline__ void rs_sched() {
    constexpr int NMF = kFI * kTJ;
    static_assert(NR <= NMF && NW <= NMF, "groups");
#pragma unroll
    for (int g = 0; g < NMF; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
        if (g < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
        if (g >= NMF - NW) {
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // LDS write
            if (LOAD) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // global load
        }
    }
}
// One k step (stage ks, buffer ks % 2) of the register-staged pipeline:
// WRITE stage ks + 1 from the registers, LOAD stage ks + 2 into them, NEXT:
// the barrier in the last substep publishes stage ks + 1 (every wave's
// writes done, every wave done reading stage ks) and its first fragments are
// read under the last MFMAs. Each substep's MFMAs run at raised wave priority,
// so the SIMD's other wave issues its memory work between them.
template <typename T, bool WRITE, bool LOAD, bool NEXT>
__device__ __forceinline__ void stage_body_rs(f32x16 (&acc)[kFI][kTJ], typename Mfma<T>::v8 (&af)[2][kFI],
                                              typename Mfma<T>::v8 (&bf)[2][kTJ], u32x4 (&r)[kLoads],
                                              const StageCtx& cx, int lane, int ks) {
    const uint8_t* st = cx.lds + (ks & 1) * kStageBytes;
    uint8_t* nst = cx.lds + ((ks + 1) & 1) * kStageBytes;
    constexpr int kG = kFI + kTJ;
    constexpr int kW = kLoads / (kSub - 1);
#pragma unroll
    for (int s = 0; s < kSub; ++s) {
        const int c = s & 1, n = c ^ 1;
        const bool last = s + 1 == kSub;
        if (!last) {
            read_frags<T>(af[n], bf[n], st, cx.fa, cx.fb, cx.slot ^ (32 * (s + 1)));
            if (WRITE) rs_write(r, nst, cx.wave, lane, rs_lo(s), rs_lo(s + 1));
            if (LOAD) rs_fetch(r, cx.wbase, cx.xbase, cx.src, ks + 2, rs_lo(s), rs_lo(s + 1));
        } else if (NEXT) {
            __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): this wave's writes landed
            __builtin_amdgcn_s_barrier();
            read_frags<T>(af[n], bf[n], nst, cx.fa, cx.fb, cx.slot);
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) acc[fi][tj] = Mfma<T>::run(af[c][fi], bf[c][tj], acc[fi][tj]);
        if (!last && WRITE) {
            if (rs_lo(s + 1) - rs_lo(s) == kW) rs_sched<kG, kW, LOAD>();
            else rs_sched<kG, kW + 1, LOAD>();
        } else if (!last || NEXT) {
            rs_sched<kG, 0, false>();
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    }
}

// Residual rows of a 16-bit gated-residual tile into LDS: 128 rows from
// `row0`, 128 / kWaves per wave (row r at r * 512 bytes, chunk c at slot
// c ^ (r % 32), the epilogue's staging layout), 2 rows per direct-to-LDS
// load: lane l fills slot l % 32 of row 2 it + l / 32. Rows past the last
// token read the last.
__device__ __forceinline__ void res_rows(const GemmArgs& a, int64_t t0, int64_t n0, uint8_t* lds, int row0, int wave,
                                         int lane) {
    constexpr int kRows = 128 / kWaves;
    const uint8_t* rb = static_cast<const uint8_t*>(a.res);
    const int64_t last = a.rows - 1;
    const int fr = lane & 31, h = lane >> 5;
#pragma unroll
    for (int it = 0; it < kRows / 2; ++it) {
        const int r = row0 + wave * kRows + it * 2 + h;
        const int64_t t = t0 + r < last ? t0 + r : last;
        const int c = fr ^ (r & 31);
        __builtin_amdgcn_global_load_lds(rb + (t * a.ldo + n0 + c * 8) * 2,
                                         lds + (row0 + wave * kRows + it * 2) * (kBF * 2), 16, 0, 0);
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

    // Load i of wave w fills the 64 chunks [(i*kWaves + w)*64, +64) of a
    // stage (weight tile first, then token tile), one 16-byte chunk per lane;
    // each lane fetches the global chunk that the swizzle puts at its slot.
    // Pad tokens read the last row.
    int64_t src[kLoads];   // byte offsets
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int p = (i * kWaves + wave) * 64 + lane;
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
    if constexpr (kRegStaged) {
        static_assert(kStages == 2, "two buffers");
        u32x4 r[kLoads];
        rs_fetch(r, wbase, xbase, src, 0, 0, kLoads);
        rs_write(r, lds, wave, lane, 0, kLoads);
        if (ksteps > 1) rs_fetch(r, wbase, xbase, src, 1, 0, kLoads);
        __builtin_amdgcn_s_waitcnt(0xC07F);      // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        V8 af[2][kFI], bf[2][kTJ];
        read_frags<T>(af[0], bf[0], lds, fa, fb, slot);
        __builtin_amdgcn_sched_barrier(0);
        const StageCtx cx{wbase, xbase, src, lds, fa, fb, slot, wave};
        int ks = 0;
        for (; ks + 2 < ksteps; ++ks) stage_body_rs<T, true, true, true>(acc, af, bf, r, cx, lane, ks);
        if (ks + 1 < ksteps) stage_body_rs<T, true, false, true>(acc, af, bf, r, cx, lane, ks++);
        if constexpr (RES_PRE) {
            // stage ks + 1's buffer: every wave finished reading it before the
            // barrier of stage ks - 1, and nothing writes it any more
            static_assert(kStageBytes == 128 * kBF * 2, "a free stage holds 128 residual rows");
            res_rows(a, t0, n0, lds, ((ks + 1) & 1) * 128, wave, lane);
        }
        stage_body_rs<T, false, false, false>(acc, af, bf, r, cx, lane, ks);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();            // every wave is done reading the stages
    } else {
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
}

#ifndef T2H_GEMM_NTS
#define T2H_GEMM_NTS 1
#endif
// A 16-byte store of an epilogue; non-temporal with T2H_GEMM_NTS (the GEMM
// never re-reads its outputs, so they need not displace operands in L2).
__device__ __forceinline__ void out_store16(void* p, u32x4 w) {
    if constexpr (T2H_GEMM_NTS) __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
    else *reinterpret_cast<u32x4*>(p) = w;
}

__device__ __forceinline__ void zero_acc(f32x16 (&acc)[kFI][kTJ]) {
#pragma unroll
    for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
        for (int tj = 0; tj < kTJ; ++tj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fi][tj][r] = 0.0f;
}

}  // namespace
}  // namespace t2h
