// One flow-matching Euler step of the sampler over a flat state x_t:
// classifier-free-guidance combine, optional CFG rescale, the Euler update and
// the x_0 prediction, in one elementwise pass (plus, for the rescale, one
// statistics pass in front of it).
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
// caller's token segments (varlen state, biased std).
//
// The rescale of a single segment on whole 16-byte vectors whose three
// tensors fit in the registers of the resident grid (the config-5 latent:
// 6.4M f32 elements, 4 vectors of each tensor per thread) takes one launch,
// euler_fused_kernel: it loads the three inputs once, publishes per-block
// sums, meets the other blocks at a grid barrier and stores (see there).
// Otherwise (several segments, larger states, a workspace without room for
// the barrier) the rescale takes two launches:
// - euler_stats_kernel: one block of 1024 threads per 16,384 elements of a
//   segment, at most kStatsMaxPerSeg, take equal shares of it, load them with
//   16-byte loads (16 elements of each tensor per thread per load group), sum
//   x0_pos, x0_pos^2, x0_cfg, x0_cfg^2 in f64 per thread, reduce through DPP
//   row sums and one LDS combine, and write one f64 partial quad per block.
//   Its loads are ordinary (cached), so the elementwise pass that re-reads
//   the same 3 tensors right after finds them in the infinity cache when
//   they fit.
// - euler_apply_kernel: each block (2048 elements) first sums its segment's
//   partials (at most kStatsMaxPerSeg quads, in a fixed order per thread)
//   into the segment's ratio,
//   with its own element loads already in flight, then runs the elementwise
//   step. Every block of a segment sums the same partials in the same order,
//   so all of them compute the same ratio bits, and the result is
//   deterministic.
// Without the rescale there is only the elementwise pass.
//
// Reference: samplers/flow_euler.mojo:56-57 (_scaled), 68-70
// (_v_to_xstart), 75-149 (_rescale_pred), 151-181 (_inference),
// 196-210 (_sample_impl step).
#include <mutex>
#include <vector>

#include "t2h_device.h"
#include "t2h_internal.h"

#ifndef T2H_EULER_NTL
#define T2H_EULER_NTL 0   // elementwise pass: non-temporal loads (measured slower: 21.9 vs 19.8 us)
#endif
#ifndef T2H_EULER_NTS
#define T2H_EULER_NTS 1   // elementwise pass: non-temporal stores
#endif

namespace t2h {
namespace {

__device__ __forceinline__ float v_to_x0(float x, float v, float a, float cc) {
    return sub_rn(mul_rn(x, a), mul_rn(v, cc));
}

// f64 DPP move of both 32-bit halves.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Wave64 sum of an f64 (all lanes active); wave-uniform result, fixed order.
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_d<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_d<0x141>(v);   // row_half_mirror
    v += dpp_d<0x140>(v);   // row_mirror
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

// Block sum of 4 f64 values (all threads of the block take part); every
// thread gets the totals, summed over the waves in wave order.
template <int NW>
__device__ __forceinline__ void block_sum4(double (&v)[4], double (*sh)[4]) {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = wave_sum_d(v[k]);
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) sh[w][k] = v[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        double s = sh[0][k];
#pragma unroll
        for (int i = 1; i < NW; ++i) s += sh[i][k];
        v[k] = s;
    }
}

// x0_pos / x0_cfg contributions of one element to the four sums.
__device__ __forceinline__ void stats_add(const EulerArgs& a, float xv, float pos, float neg, double (&acc)[4]) {
    const float pred = add_rn(mul_rn(pos, a.gp), mul_rn(neg, a.gn));
    const double x0p = v_to_x0(xv, pos, a.a, a.cc);
    const double x0c = v_to_x0(xv, pred, a.a, a.cc);
    acc[0] += x0p;
    acc[1] += x0p * x0p;   // exact: a product of two f32 fits an f64
    acc[2] += x0c;
    acc[3] += x0c * x0c;
}

template <typename T>
__global__ __launch_bounds__(kStatsBlock) void euler_stats_kernel(EulerArgs a) {
    constexpr int NW = kStatsBlock / 64;
    __shared__ double sh[NW][4];
    const int64_t b = block_linear();
    if (b >= a.nstats) return;   // block-uniform
    int64_t j, per, lo, hi;
    if (a.uniform) {
        per = a.pper;
        const int64_t s = b / per;
        j = b - s * per;
        lo = s * a.row_size;
        hi = lo + a.row_size;
    } else {
        int s = 0;
        while (s + 1 < a.nseg && a.pbase[s + 1] <= b) ++s;
        j = b - a.pbase[s];
        per = a.pbase[s + 1] - a.pbase[s];
        lo = a.bounds[s];
        hi = a.bounds[s + 1];
    }
    // the segment's `per` blocks take equal shares of whole vectors
    constexpr int V = kPack<T>;
    const int64_t share = ((hi - lo + V - 1) / V + per - 1) / per * V;
    const int64_t c0 = lo + j * share;
    const int64_t c1 = c0 + share < hi ? c0 + share : hi;
    const T* __restrict__ x = static_cast<const T*>(a.x);
    const T* __restrict__ vp = static_cast<const T*>(a.v_pos);
    const T* __restrict__ vn = static_cast<const T*>(a.v_neg);
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    if (a.vec) {
        // c0 and c1 are multiples of V: every vector lies inside [c0, c1);
        // a group's loads past c1 are clamped to the last vector
        // (unconditional loads stay in flight together) and not summed
        constexpr int NV = kStatsPer / V;
        for (int64_t g0 = c0; g0 < c1; g0 += (int64_t)kStatsBlock * V * NV) {
            float xv[NV][V], pv[NV][V], nv[NV][V];
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int64_t e = g0 + ((int64_t)i * kStatsBlock + threadIdx.x) * V;
                const int64_t el = e < c1 ? e : c1 - V;
                load_elems<T, V>(x + el, xv[i]);
                load_elems<T, V>(vp + el, pv[i]);
                load_elems<T, V>(vn + el, nv[i]);
            }
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int64_t e = g0 + ((int64_t)i * kStatsBlock + threadIdx.x) * V;
                if (e < c1) {
#pragma unroll
                    for (int k = 0; k < V; ++k) stats_add(a, xv[i][k], pv[i][k], nv[i][k], acc);
                }
            }
        }
    } else {
        for (int64_t e = c0 + threadIdx.x; e < c1; e += kStatsBlock)
            stats_add(a, ld1(x + e), ld1(vp + e), ld1(vn + e), acc);
    }
    block_sum4<NW>(acc, sh);
    if (threadIdx.x == 0) {
        double* p = a.partial + b * 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) p[k] = acc[k];
    }
}

// std(x0_pos) / std(x0_cfg) of a segment of m elements from its four sums:
// unbiased for a dense row, biased (mean(x^2) - mean(x)^2) for a varlen
// segment.
__device__ __forceinline__ float ratio_of_sums(const double (&acc)[4], int64_t m, bool unbiased) {
    const double md = (double)m;
    double vp, vc;
    if (unbiased) {
        vp = (acc[1] - acc[0] * (acc[0] / md)) / (md - 1.0);
        vc = (acc[3] - acc[2] * (acc[2] / md)) / (md - 1.0);
    } else {
        vp = acc[1] / md - (acc[0] / md) * (acc[0] / md);
        vc = acc[3] / md - (acc[2] / md) * (acc[2] / md);
    }
    if (unbiased && m == 1) return __builtin_nanf("");   // 0/0 as the reference's m - 1 = 0
    return (float)(sqrt(vp > 0.0 ? vp : 0.0) / sqrt(vc > 0.0 ? vc : 0.0));
}

// The rescale ratio of segment s from its partials (called by every thread
// of a kEulerBlock-thread block; the same bits in every block).
__device__ __forceinline__ float segment_ratio(const EulerArgs& a, int s, double (*sh)[4]) {
    int64_t p0, np, m;
    if (a.uniform) {
        p0 = (int64_t)s * a.pper;
        np = a.pper;
        m = a.row_size;
    } else {
        p0 = a.pbase[s];
        np = a.pbase[s + 1] - p0;
        m = a.bounds[s + 1] - a.bounds[s];
    }
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int64_t i = threadIdx.x; i < np; i += kEulerBlock) {   // fixed order per thread
        const double2* q = reinterpret_cast<const double2*>(a.partial + (p0 + i) * 4);
        const double2 u = q[0], w = q[1];
        acc[0] += u.x; acc[1] += u.y; acc[2] += w.x; acc[3] += w.y;
    }
    block_sum4<kEulerBlock / 64>(acc, sh);
    return ratio_of_sums(acc, m, a.uniform != 0);
}

template <int MODE>
__device__ __forceinline__ void apply_elem(const EulerArgs& a, float ratio, float xv, float pos, float neg,
                                           float& xprev, float& x0) {
    float pred = MODE == 0 ? pos : add_rn(mul_rn(pos, a.gp), mul_rn(neg, a.gn));
    if (MODE == 2) {
        const float x0c = v_to_x0(xv, pred, a.a, a.cc);
        const float x0r = mul_rn(x0c, ratio);
        const float x0b = add_rn(mul_rn(a.gr, x0r), mul_rn(a.one_m_gr, x0c));
        pred = __fdiv_rn(sub_rn(mul_rn(a.a, xv), x0b), a.cc);
    }
    xprev = sub_rn(xv, mul_rn(pred, a.dt));
    x0 = v_to_x0(xv, pred, a.a, a.cc);
}

template <typename T, int MODE>
__global__ __launch_bounds__(kEulerBlock) void euler_apply_kernel(EulerArgs a) {
    __shared__ double sh[kEulerBlock / 64][4];
    const T* __restrict__ x = static_cast<const T*>(a.x);
    const T* __restrict__ vp = static_cast<const T*>(a.v_pos);
    const T* __restrict__ vn = static_cast<const T*>(a.v_neg);
    T* __restrict__ xp = static_cast<T*>(a.x_prev);
    T* __restrict__ x0o = static_cast<T*>(a.pred_x0);
    const int64_t b = block_linear();
    if (b >= a.nblocks) return;   // block-uniform
    int s = 0;
    int64_t lo, hi;
    if (MODE == 2) {
        int64_t j;
        if (a.uniform) {
            const int64_t nb = (a.row_size + kEulerChunk - 1) / kEulerChunk;
            s = (int)(b / nb);
            j = b - (int64_t)s * nb;
            lo = (int64_t)s * a.row_size + j * kEulerChunk;
            hi = (int64_t)(s + 1) * a.row_size;
        } else {
            while (s + 1 < a.nseg && a.blk_base[s + 1] <= b) ++s;
            j = b - a.blk_base[s];
            lo = a.bounds[s] + j * kEulerChunk;
            hi = a.bounds[s + 1];
        }
    } else {
        lo = b * kEulerChunk;
        hi = a.n;
    }
    hi = lo + kEulerChunk < hi ? lo + kEulerChunk : hi;

    if (a.vec) {
        constexpr int V = kPack<T>;
        constexpr int NV = kEulerChunk / kEulerBlock / V;
        float xv[NV][V], pv[NV][V], nv[NV][V];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int64_t e = lo + ((int64_t)i * kEulerBlock + threadIdx.x) * V;
            const int64_t el = e < hi ? e : hi - V;
            load_elems<T, V, T2H_EULER_NTL>(x + el, xv[i]);
            load_elems<T, V, T2H_EULER_NTL>(vp + el, pv[i]);
            if (MODE != 0) load_elems<T, V, T2H_EULER_NTL>(vn + el, nv[i]);
        }
        const float ratio = MODE == 2 ? segment_ratio(a, s, sh) : 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int64_t e = lo + ((int64_t)i * kEulerBlock + threadIdx.x) * V;
            float o[V], z[V];
#pragma unroll
            for (int k = 0; k < V; ++k)
                apply_elem<MODE>(a, ratio, xv[i][k], pv[i][k], MODE != 0 ? nv[i][k] : 0.0f, o[k], z[k]);
            if (e < hi) {
                store_elems<T, V, T2H_EULER_NTS>(xp + e, o);
                if (x0o != nullptr) store_elems<T, V, T2H_EULER_NTS>(x0o + e, z);
            }
        }
    } else {
        const float ratio = MODE == 2 ? segment_ratio(a, s, sh) : 0.0f;
        for (int64_t e = lo + threadIdx.x; e < hi; e += kEulerBlock) {
            float o, z;
            apply_elem<MODE>(a, ratio, ld1(x + e), ld1(vp + e), MODE != 0 ? ld1(vn + e) : 0.0f, o, z);
            st1(xp + e, o);
            if (x0o != nullptr) st1(x0o + e, z);
        }
    }
}

// The one-launch rescale over a single segment [fuse_lo, fuse_hi) of whole
// 16-byte vectors. Each data block holds KV vectors of each tensor per
// thread, in registers, from the first load to the last store:
// 1. load x, v_pos, v_neg; sum the block's four x0 sums (f64, fixed order),
//    publish them as the block's partial quad and raise the block's flag;
// 2. one extra block, which holds no vectors, waits for every flag, sums
//    the quads in a fixed order into the ratio (the same bits on every
//    call) and publishes it in 8 release slots, 128 bytes apart, which the
//    data blocks poll in turn (block b polls slot b % 8);
// 3. every data block applies the step to the vectors it holds and stores.
// In the normal course no two blocks update one word (same-address atomics
// from ~1,600 blocks serialize). Each slot carries a 64-bit epoch: a launch reads it (e), its
// blocks raise their flags to e + 1 and the reducing block sets the slot
// to e + 1. Flags left by earlier launches hold at most e, so the
// workspace needs no clearing and a graph replay reads the epoch the last
// launch left; a first use on uninitialised memory is safe unless a word
// happens to hold e + 1 (64-bit values: chance 2^-64 per word). The ratio
// goes out in the slot's release word, with the new epoch's low half, in
// one 64-bit store; a data block waits for that word to differ from what it
// read at its start (the epoch half always does), so one load brings it
// the release and the ratio together.
// The launcher sizes the grid to be resident at once (occupancy x CUs). A
// grid that is not (other streams' kernels hold part of the GPU) still
// finishes with the same result: a data block that has waited fuse_polls
// polls for the ratio marks its vectors left and exits, which frees its
// slot for the blocks not yet running; the reducing block then loads the
// left vectors from memory and stores them. A block that sees the ratio
// right after marking takes its vectors back; one exchange on the block's
// claim word decides which of the two stores them, so no vector is
// computed twice (x_prev may alias x_t). The reducing block's own wait is
// bounded too (2^20 polls, about a second): past it, it sets `err` and goes
// on, so the grid always drains.
struct EulerSlot {
    uint64_t epoch;   // e at the launch, e + 1 after it
    uint64_t word;    // the release word: low 32 bits of the epoch (high
                      // half) and the ratio's bits (low half)
    unsigned pad[28];
};
__device__ __forceinline__ uint64_t release_word(uint64_t epoch, float ratio) {
    return ((uint64_t)(uint32_t)epoch << 32) | __builtin_bit_cast(uint32_t, ratio);
}
struct EulerBar {
    uint64_t err;     // set to e + 1 by the reducing block if it stopped waiting
    uint64_t pad[7];
    EulerSlot slot[8];
    uint64_t flag[kFuseMaxBlocks];    // e + 1 of the block's slot once its quad is out
    uint64_t leave[kFuseMaxBlocks];   // e + 1 once the block has stopped waiting for the ratio
    uint64_t claim[kFuseMaxBlocks];   // exchanged to e + 1 by whoever stores a left block's vectors
};
static_assert(sizeof(EulerSlot) == 128, "one slot per 128 bytes");
static_assert(sizeof(EulerBar) == kEulerBarBytes, "barrier words");

__device__ __forceinline__ uint64_t shared_load(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void shared_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// true for the first caller of a launch (the word held anything but v)
__device__ __forceinline__ bool claim_first(uint64_t* p, uint64_t v) {
    return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != v;
}

template <typename T>
__device__ __forceinline__ void unpack16(const u32x4& w, float* f) {
    constexpr int WN = Word<T>::N;
    Word<T>::unpack(w.x, f);
    Word<T>::unpack(w.y, f + WN);
    Word<T>::unpack(w.z, f + 2 * WN);
    Word<T>::unpack(w.w, f + 3 * WN);
}

template <typename T>
__device__ __forceinline__ u32x4 pack16(const float* f) {
    constexpr int WN = Word<T>::N;
    u32x4 w;
    w.x = Word<T>::pack(f);
    w.y = Word<T>::pack(f + WN);
    w.z = Word<T>::pack(f + 2 * WN);
    w.w = Word<T>::pack(f + 3 * WN);
    return w;
}

constexpr int kFusePolls = 1 << 20;   // the reducing block's wait for the flags, at most

// Every word the blocks of euler_fused_kernel share (partial quads, flags,
// release slots, leave marks, claims) is written and read as a device-scope
// relaxed atomic: a
// device-coherent access that no XCD's L2 holds stale. The wave's own stores
// are ordered by waiting for them before the store that publishes them (no
// agent-scope fence: its L2 write-back and invalidate would run on every
// block's L2 and cost more than the step). The readers issue their loads
// after the load that saw the flag.
__device__ __forceinline__ double shared_load(const double* p) {
    return __hip_atomic_load(const_cast<double*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_after_stores() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");   // no compiler reordering across it
    __builtin_amdgcn_s_waitcnt(0x0F70);                      // vmcnt(0): the wave's stores are done
}

template <typename T, int KV>
__global__ __launch_bounds__(kFuseBlock) void euler_fused_kernel(EulerArgs a) {
    constexpr int V = kPack<T>;
    constexpr int NW = kFuseBlock / 64;
    constexpr int NJ = kFuseMaxBlocks / kFuseBlock;   // block-index groups a reducing thread covers
    __shared__ double sh[NW][4];
    __shared__ float ratio_s;
    __shared__ unsigned own_s;                        // data block: 1 = store the held vectors
    __shared__ unsigned long long left_s[NJ][NW];    // reducing block: ballots of the left blocks
    __shared__ uint64_t want_s[8];                   // reducing block: each slot's new epoch
    EulerBar* bar = static_cast<EulerBar*>(a.fuse_ws);
    double* partial = reinterpret_cast<double*>(static_cast<char*>(a.fuse_ws) + kEulerBarBytes);
    const unsigned nblk = gridDim.x - 1;   // data blocks; the last block reduces
    const int64_t nv = (a.fuse_hi - a.fuse_lo) / V;
    // buffer descriptors over the segment: a 32-bit byte offset per vector
    // serves the three tensors and the two outputs, and the descriptor's
    // range check (on the offset register) makes loads past the segment read
    // 0 and drops stores past it
    const int bytes = (int)(nv * 16);
    auto rsrc = [&](const void* p) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(static_cast<const T*>(p) + a.fuse_lo), 0, bytes,
                                                 0x00020000);
    };
    // vector k of this thread in data block blk
    auto vec = [&](unsigned blk, int k) { return (int64_t)blk * kFuseBlock * KV + k * kFuseBlock + threadIdx.x; };
    auto load_block = [&](unsigned blk, u32x4 (&xw)[KV], u32x4 (&pw)[KV], u32x4 (&nw)[KV]) {
        const __amdgpu_buffer_rsrc_t rx = rsrc(a.x), rp = rsrc(a.v_pos), rn = rsrc(a.v_neg);
#pragma unroll
        for (int k = 0; k < KV; ++k) {
            // non-temporal (aux 2): each vector is read once (26.2 against
            // 27.7 us with the default policy, config-5 latent)
            const int off = (int)(vec(blk, k) * 16);
            xw[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 2);
            pw[k] = __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, 2);
            nw[k] = __builtin_amdgcn_raw_buffer_load_b128(rn, off, 0, 2);
        }
    };
    auto store_block = [&](unsigned blk, float ratio, const u32x4 (&xw)[KV], const u32x4 (&pw)[KV],
                           const u32x4 (&nw)[KV]) {
        const __amdgpu_buffer_rsrc_t ro = rsrc(a.x_prev);
        const __amdgpu_buffer_rsrc_t rz = rsrc(a.pred_x0 != nullptr ? a.pred_x0 : a.x_prev);
        constexpr int kStoreAux = T2H_EULER_NTS ? 2 : 0;   // 2: the non-temporal bit
#pragma unroll
        for (int k = 0; k < KV; ++k) {
            if (vec(blk, k) < nv) {
                float xf[V], pf[V], nf[V], o[V], z[V];
                unpack16<T>(xw[k], xf);
                unpack16<T>(pw[k], pf);
                unpack16<T>(nw[k], nf);
#pragma unroll
                for (int i = 0; i < V; ++i) apply_elem<2>(a, ratio, xf[i], pf[i], nf[i], o[i], z[i]);
                const int off = (int)(vec(blk, k) * 16);
                __builtin_amdgcn_raw_buffer_store_b128(pack16<T>(o), ro, off, 0, kStoreAux);
                if (a.pred_x0 != nullptr) __builtin_amdgcn_raw_buffer_store_b128(pack16<T>(z), rz, off, 0, kStoreAux);
            }
        }
    };

    if (blockIdx.x == nblk) {
        // wait for every data block's flag, sum their quads in a fixed order
        // (the same bits on every call), publish the ratio. The blocks this
        // thread looks at (i = threadIdx.x + j * kFuseBlock) all belong to
        // slot threadIdx.x % 8.
        const uint64_t want = shared_load(&bar->slot[threadIdx.x % 8].epoch) + 1;
        if (threadIdx.x < 8) want_s[threadIdx.x] = want;
        double t[4] = {0.0, 0.0, 0.0, 0.0};
        bool all = false;
        for (int it = 0; it < kFusePolls && !all; ++it) {
            uint64_t f[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                // every flag load in flight at once: unconditional, indices
                // past the last data block read its flag again and ignore it
                // (its slot, and so its epoch, can differ from this thread's)
                const unsigned i = threadIdx.x + j * kFuseBlock;
                f[j] = shared_load(&bar->flag[i < nblk ? i : nblk - 1]);
            }
            int missing = 0;
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                missing += (threadIdx.x + j * kFuseBlock < nblk && f[j] != want) ? 1 : 0;
            all = __syncthreads_and(missing == 0) != 0;
            if (!all) __builtin_amdgcn_s_sleep(1);
        }
        if (!all && threadIdx.x == 0) shared_store(&bar->err, want);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        for (unsigned i0 = threadIdx.x; i0 < nblk; i0 += 4 * kFuseBlock) {
            // quads i0, i0 + kFuseBlock, ... in that (fixed) order, four loads
            // in flight at once
            double q[4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const unsigned i = i0 + u * kFuseBlock;
                const double* p = partial + (int64_t)(i < nblk ? i : nblk - 1) * 4;
#pragma unroll
                for (int c = 0; c < 4; ++c) q[u][c] = shared_load(p + c);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (i0 + u * kFuseBlock < nblk) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) t[c] += q[u][c];
                }
            }
        }
        block_sum4<NW>(t, sh);
        if (threadIdx.x < 8) {
            const float r = ratio_of_sums(t, a.fuse_hi - a.fuse_lo, a.uniform != 0);
            if (threadIdx.x == 0) ratio_s = r;
            // the ratio and the new epoch's low half in one 64-bit store:
            // a block that sees the word change holds the ratio with it
            shared_store(&bar->slot[threadIdx.x].word, release_word(want, r));
            shared_store(&bar->slot[threadIdx.x].epoch, want);
            publish_after_stores();   // the ratio is out before the leave marks are read
        }
        __syncthreads();
        // blocks that stopped waiting before the ratio was out: leave marks
        // four groups at a time (this block's scan is off the data blocks'
        // path: they have the ratio), one ballot per wave and group
#pragma unroll 4
        for (int j = 0; j < NJ; ++j) {
            const unsigned i = threadIdx.x + j * kFuseBlock;
            const uint64_t m = shared_load(&bar->leave[i < nblk ? i : nblk - 1]);
            const unsigned long long b = __ballot(i < nblk && m == want);
            if ((threadIdx.x & 63) == 0) left_s[j][threadIdx.x >> 6] = b;
        }
        __syncthreads();
        const float ratio = ratio_s;
#pragma unroll 1
        for (int j = 0; j < NJ; ++j) {
#pragma unroll 1
            for (int w = 0; w < NW; ++w) {
                for (unsigned long long m = left_s[j][w]; m != 0; m &= m - 1) {   // block-uniform
                    const unsigned blk = (unsigned)(j * kFuseBlock + w * 64 + __builtin_ctzll(m));
                    __shared__ unsigned mine_s;
                    if (threadIdx.x == 0) mine_s = claim_first(&bar->claim[blk], want_s[blk % 8]) ? 1u : 0u;
                    __syncthreads();
                    const bool take = mine_s != 0;
                    __syncthreads();
                    if (take) {
                        u32x4 xw[KV], pw[KV], nw[KV];
                        load_block(blk, xw, pw, nw);
                        store_block(blk, ratio, xw, pw, nw);
                    }
                }
            }
        }
        return;
    }

    EulerSlot* sl = &bar->slot[blockIdx.x % 8];
    uint64_t e0 = 0, w0 = 0;   // the slot's epoch and release word at the launch
    if (threadIdx.x == 0) {
        e0 = shared_load(&sl->epoch);
        w0 = shared_load(&sl->word);
    }
    u32x4 xw[KV], pw[KV], nw[KV];
    load_block(blockIdx.x, xw, pw, nw);
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int k = 0; k < KV; ++k) {
        if (vec(blockIdx.x, k) < nv) {
            float xf[V], pf[V], nf[V];
            unpack16<T>(xw[k], xf);
            unpack16<T>(pw[k], pf);
            unpack16<T>(nw[k], nf);
#pragma unroll
            for (int i = 0; i < V; ++i) stats_add(a, xf[i], pf[i], nf[i], acc);
        }
    }
    // the block's quad: wave sums, then lanes 0-3 of wave 0 add the waves'
    // values in wave order (few registers beside the held vectors)
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const double t = wave_sum_d(acc[c]);
        if ((threadIdx.x & 63) == 0) sh[w][c] = t;
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        double q = sh[0][threadIdx.x];
#pragma unroll
        for (int i = 1; i < NW; ++i) q += sh[i][threadIdx.x];
        __hip_atomic_store(partial + (int64_t)blockIdx.x * 4 + threadIdx.x, q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        publish_after_stores();   // the quad is out before the flag
        if (threadIdx.x == 0) shared_store(&bar->flag[blockIdx.x], e0 + 1);
    }
    if (threadIdx.x == 0) {
        bool done = false;
        uint64_t w = w0;
        for (int it = 0; it < a.fuse_polls && !done; ++it) {
            w = shared_load(&sl->word);
            done = w != w0;
            if (!done) __builtin_amdgcn_s_sleep(2);
        }
        bool own = done;
        if (!done) {
            // leave the vectors to the reducing block; if the ratio is out by
            // the time the mark is, take them back unless it has claimed them
            shared_store(&bar->leave[blockIdx.x], e0 + 1);
            publish_after_stores();   // the mark is out before the ratio is looked at again
            w = shared_load(&sl->word);
            done = w != w0;
            own = done && claim_first(&bar->claim[blockIdx.x], e0 + 1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        own_s = own ? 1u : 0u;
        if (own) ratio_s = __builtin_bit_cast(float, (uint32_t)w);
    }
    __syncthreads();
    if (own_s == 0) return;   // the reducing block stores this block's vectors
    const float ratio = ratio_s;
    // only the loaded words stay live across the barrier: the products the
    // statistics formed are formed again (kept, they would double the
    // registers a thread holds and halve the resident grid)
#pragma unroll
    for (int k = 0; k < KV; ++k) asm volatile("" : "+v"(xw[k]), "+v"(pw[k]), "+v"(nw[k]));
    store_block(blockIdx.x, ratio, xw, pw, nw);
}

// Blocks of euler_fused_kernel<T, KV> resident at once on this device.
template <typename T, int KV>
int64_t fused_capacity() {
    static const int64_t cap = [] {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, euler_fused_kernel<T, KV>, kFuseBlock, 0) !=
                hipSuccess || nb <= 0)
            return (int64_t)0;
        return (int64_t)nb * device_cu_count();
    }();
    return cap;
}

template <typename T, int KV>
bool try_fused(const EulerArgs& a, hipStream_t st) {
    const int64_t nv = (a.fuse_hi - a.fuse_lo) / kPack<T>;
    const int64_t g = (nv + (int64_t)kFuseBlock * KV - 1) / ((int64_t)kFuseBlock * KV);
    if (g > kFuseMaxBlocks || g + 1 > fused_capacity<T, KV>()) return false;
    hipLaunchKernelGGL((euler_fused_kernel<T, KV>), dim3((unsigned)(g + 1)), dim3(kFuseBlock), 0, st, a);
    return true;
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
hipError_t launch_typed(const EulerArgs& a, int64_t cover_lo, int64_t cover_hi, hipStream_t st) {
    if (a.mode == 2) {
        // one launch when the segment fits the resident grid with 1, 2, 4 or
        // 8 vectors of each tensor per thread; else the statistics pass and
        // the elementwise pass
        const bool fused = a.fuse && a.fuse_hi > a.fuse_lo &&
                           (try_fused<T, 1>(a, st) || try_fused<T, 2>(a, st) || try_fused<T, 4>(a, st) ||
                            try_fused<T, 8>(a, st));
        if (!fused && a.nblocks > 0) {
            hipLaunchKernelGGL(euler_stats_kernel<T>, grid_1d(a.nstats), dim3(kStatsBlock), 0, st, a);
            hipLaunchKernelGGL((euler_apply_kernel<T, 2>), grid_1d(a.nblocks), dim3(kEulerBlock), 0, st, a);
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
    } else if (a.mode == 1) {
        hipLaunchKernelGGL((euler_apply_kernel<T, 1>), grid_1d(a.nblocks), dim3(kEulerBlock), 0, st, a);
    } else {
        hipLaunchKernelGGL((euler_apply_kernel<T, 0>), grid_1d(a.nblocks), dim3(kEulerBlock), 0, st, a);
    }
    return hipGetLastError();
}

// The built-in statistics scratch of t2h_flow_euler_step_noalloc: f64
// partial quads for up to kEulerScratchPartials statistics blocks (512 KB),
// one copy per GPU at its own address, held until the process ends. Host
// code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): euler_scratch() looks the device address
// up with hipGetSymbolAddress once per device and every launch takes that.
// Every statistics block writes its quad before the elementwise pass reads
// it, and the one-launch form's barrier words work from any contents, so
// nothing has to start at zero; calls that overlap on one GPU share the
// array and race.
__device__ __align__(256) double scratch[kEulerScratchPartials * 4];

}  // namespace

hipError_t euler_scratch(double** out) {
    static std::mutex mu;
    static std::vector<double*> ptrs;   // per device ordinal
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(mu);
    if (dev < (int)ptrs.size() && ptrs[dev] != nullptr) {
        *out = ptrs[dev];
        return hipSuccess;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));   // with `dev` current
    if (e != hipSuccess) return e;
    if (dev >= (int)ptrs.size()) ptrs.resize(dev + 1, nullptr);
    ptrs[dev] = static_cast<double*>(p);
    *out = ptrs[dev];
    return hipSuccess;
}

hipError_t launch_euler(const EulerArgs& a, int64_t cover_lo, int64_t cover_hi, hipStream_t s) {
    switch (a.dtype) {
        case T2H_F32: return launch_typed<float>(a, cover_lo, cover_hi, s);
        case T2H_F16: return launch_typed<_Float16>(a, cover_lo, cover_hi, s);
        default: return launch_typed<__bf16>(a, cover_lo, cover_hi, s);
    }
}

}  // namespace t2h
