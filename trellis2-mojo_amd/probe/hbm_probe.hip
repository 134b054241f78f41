// HBM streaming probes: the access patterns of the per-token kernels with
// nothing else in them, to bound what a kernel of each shape can reach on
// MI355X. Not part of libt2h; bench.py --probe times them, and rocprofv3
// counters on the same command explain the differences.
//
// Every probe streams an f16 tensor [rows, 6144] (the GELU tensor of the
// config-5 chain: one row = 768 lanes x 16 B) with non-temporal 16-byte
// loads and stores:
//   copy       y = x (one bit flipped so the data is touched)
//   gelu       y = GELU-tanh(x)
//   gelu+bias  y = GELU-tanh(x + bias[col]), bias f32 [6144], 32 B per thread
// A block has W threads and covers W * 8 columns of RPT rows (each thread
// moves RPT rows of 16 B); the 768 / W column tiles of a row tile are
// consecutive blocks. The logical blocks are dealt to P contiguous fronts
// (physical block b runs logical block (b % P) * per + b / P; front f runs
// on XCD f % 8), P = 1 is the plain order. ORDER 0 issues a thread's RPT
// loads before its stores, ORDER 1 loads and stores row by row; MAP 1 gives
// a block the rows b + k * (row tiles) instead of b * RPT + k.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kVpr = 768;   // 16-byte vectors per row

// An empty asm that claims to read `dep` and rewrite `x`: the compiler must
// wait for the load that produced `dep` before it uses `x`, and `x` keeps its
// value.
template <typename X>
__device__ __forceinline__ void fake_dep(X& x, uint32_t dep) {
    asm volatile("" : "+v"(x) : "v"(dep));
}

__device__ __forceinline__ float gelu(float v) {
    constexpr float k0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
    constexpr float k1 = k0 * 0.044715f;
    const float arg = v * __builtin_fmaf(k1, v * v, k0);
    return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(arg));
}

template <bool BIAS>
__device__ __forceinline__ u32x4 gelu8(u32x4 w, const float* b) {
    const uint32_t in[4] = {w.x, w.y, w.z, w.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(in[i] & 0xFFFFu));
        float hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(in[i] >> 16));
        if (BIAS) {
            lo = __builtin_fmaf(lo, 1.0f, b[2 * i]);
            hi = __builtin_fmaf(hi, 1.0f, b[2 * i + 1]);
        }
        lo = gelu(lo);
        hi = gelu(hi);
        o[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
    }
    return (u32x4){o[0], o[1], o[2], o[3]};
}

// KIND 0 copy, 1 gelu + bias, 2 gelu
template <int W, int RPT, int KIND, int P, int ORDER, int MAP>
__global__ __launch_bounds__(W) void stream_probe(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                  const float* __restrict__ bias, int64_t rows, int64_t nb,
                                                  int64_t per) {
    constexpr int kTiles = kVpr / W;
    const int64_t b = (int64_t)(blockIdx.x % P) * per + blockIdx.x / P;
    if (b >= nb) return;
    const int64_t rt = b / kTiles;
    const int c = (int)(b - rt * kTiles) * W + threadIdx.x;
    const int64_t nrt = nb / kTiles;
    auto row = [&](int k) -> int64_t { return MAP == 0 ? rt * RPT + k : rt + k * nrt; };
    float bv[8];
    if (KIND == 1) {
        const float4* q = reinterpret_cast<const float4*>(bias + c * 8);
        const float4 a0 = q[0], a1 = q[1];
        bv[0] = a0.x; bv[1] = a0.y; bv[2] = a0.z; bv[3] = a0.w;
        bv[4] = a1.x; bv[5] = a1.y; bv[6] = a1.z; bv[7] = a1.w;
    }
    auto apply = [&](u32x4 w) -> u32x4 {
        if (KIND == 0) {
            w.x ^= 0x3C003C00u;
            return w;
        }
        return gelu8<KIND == 1>(w, bv);
    };
    if (ORDER == 0) {
        u32x4 v[RPT];
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            const int64_t r = row(k) < rows ? row(k) : rows - 1;
            v[k] = __builtin_nontemporal_load(src + r * kVpr + c);
        }
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            if (row(k) >= rows) break;
            __builtin_nontemporal_store(apply(v[k]), dst + row(k) * kVpr + c);
        }
    } else {
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            if (row(k) >= rows) break;
            const u32x4 v = __builtin_nontemporal_load(src + row(k) * kVpr + c);
            __builtin_nontemporal_store(apply(v), dst + row(k) * kVpr + c);
        }
    }
}

template <int W, int RPT, int KIND, int P, int ORDER = 0, int MAP = 0>
int launch(const void* s, void* d, const float* bias, int64_t rows, hipStream_t st) {
    const int64_t nb = (rows + RPT - 1) / RPT * (kVpr / W);
    const int64_t per = (nb + P - 1) / P;
    hipLaunchKernelGGL((stream_probe<W, RPT, KIND, P, ORDER, MAP>), dim3((unsigned)(per * P)), dim3(W), 0, st,
                       static_cast<const u32x4*>(s), static_cast<u32x4*>(d), bias, rows, nb, per);
    return (int)hipGetLastError();
}

// Head-major fan-out (the attention pack's write pattern): the [rows, 6144]
// tensor is read as 4 slabs of 1536 columns (12 heads of 128 f16 = 256 B);
// a block is 8 waves over 8 rows of one slab, one wave per row (3 x 1 KB
// loads per wave). MODE 0 stores the rows back row-major (the contiguous
// baseline); MODE 1 stores each head's 256 B straight into plane
// [48 planes][rows][128], so one wave store covers 4 planes; MODE 2 stages
// the 8 rows in LDS and stores 4 rows x 256 B of one plane per wave store,
// 1 KB contiguous.
// MODE 3 and 4 are MODE 0 and 1 with the waves of a block on 8 consecutive
// (row, slab) pieces in memory order (2 whole rows, 24 KB contiguous)
// instead of one slab of 8 rows (8 pieces 12 KB apart).
template <int MODE>
__global__ __launch_bounds__(512) void headmajor_probe(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                       int64_t rows) {
    constexpr int kPitch = 1536 / 8 + 1;   // 16-byte vectors per LDS row (+1 against bank conflicts)
    __shared__ u32x4 lds[MODE == 2 ? 8 * kPitch : 1];
    const int64_t b = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t piece = b * 8 + wave;
    const int slab = MODE >= 3 ? (int)(piece & 3) : (int)(b & 3);
    const int64_t tile = b >> 2;
    const int64_t r = MODE >= 3 ? piece >> 2 : tile * 8 + wave;
    const int64_t rl = r < rows ? r : rows - 1;
    u32x4 v[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) v[j] = __builtin_nontemporal_load(src + rl * kVpr + slab * 192 + j * 64 + lane);
#pragma unroll
    for (int j = 0; j < 3; ++j) v[j].x ^= 0x3C003C00u;
    if (MODE == 0 || MODE == 3) {
        if (r < rows) {
#pragma unroll
            for (int j = 0; j < 3; ++j) __builtin_nontemporal_store(v[j], dst + r * kVpr + slab * 192 + j * 64 + lane);
        }
    } else if (MODE == 1 || MODE == 4) {
        if (r < rows) {
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const int plane = slab * 12 + j * 4 + (lane >> 4);
                __builtin_nontemporal_store(v[j], dst + ((int64_t)plane * rows + r) * 16 + (lane & 15));
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 3; ++j) lds[wave * kPitch + j * 64 + lane] = v[j];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int i = wave * 3 + j;          // 24 plane stores per block
            const int h = i >> 1;                // head within the slab
            const int rr = (i & 1) * 4 + (lane >> 4);
            const int64_t row = tile * 8 + rr;
            const u32x4 w = lds[rr * kPitch + h * 16 + (lane & 15)];
            if (row < rows)
                __builtin_nontemporal_store(w, dst + ((int64_t)(slab * 12 + h) * rows + row) * 16 + (lane & 15));
        }
    }
}

template <int MODE>
int launch_hm(const void* s, void* d, const float*, int64_t rows, hipStream_t st) {
    const int64_t nb = (rows + 7) / 8 * 4;
    hipLaunchKernelGGL((headmajor_probe<MODE>), dim3((unsigned)nb), dim3(512), 0, st, static_cast<const u32x4*>(s),
                       static_cast<u32x4*>(d), rows);
    return (int)hipGetLastError();
}

typedef int (*Launch)(const void*, void*, const float*, int64_t, hipStream_t);
// One 16-byte vector per thread (one row per thread), with the bias shared
// by the rows of a block through LDS: a block is RPB rows x WPR waves per
// row, covering a column slab of WPR * 512 elements (1 KB per wave, 12 / WPR
// slabs per row, slab-fastest block order dealt to P fronts). KIND 1 loads
// the slab's f32 bias once per block (16 B per thread of the first
// WPR * 128) into LDS behind an LDS-only barrier that leaves the row load in
// flight; every thread then reads its 32 B of bias from LDS.
// P = 0: a 2-D grid (x = slab, y = row tile) instead of the 1-D block index.
template <int WPR, int RPB, int KIND, int P>
__global__ __launch_bounds__(WPR * RPB * 64) void slab_probe(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                            const float* __restrict__ bias, int64_t rows,
                                                            int64_t nb, int64_t per) {
    static_assert(RPB >= 2 && 12 % WPR == 0, "shape");
    constexpr int S = 12 / WPR;       // column slabs per row
    constexpr int SV = WPR * 64;      // 16-byte vectors per slab row
    constexpr bool kBias = KIND == 1 || KIND == 3;   // KIND 2 / 3: copy / gelu+bias behind a lead load
    __shared__ float4 bl[kBias ? 2 * SV : 1];
    const int64_t b = P == 0 ? (int64_t)blockIdx.y * S + blockIdx.x
                             : (int64_t)(blockIdx.x % P) * per + blockIdx.x / P;
    if (b >= nb) return;   // block-uniform, before the barrier
    const int slab = P == 0 ? (int)blockIdx.x : (int)(b % S);
    const int64_t tile = P == 0 ? (int64_t)blockIdx.y : b / S;
    const int wave = threadIdx.x >> 6;
    const int j = (wave % WPR) * 64 + (threadIdx.x & 63);   // vector within the slab row
    const int64_t r = tile * RPB + wave / WPR;
    const int c = slab * SV + j;
    float4 bq = {0.f, 0.f, 0.f, 0.f};
    if (kBias && threadIdx.x < 2 * SV) bq = reinterpret_cast<const float4*>(bias)[slab * 2 * SV + threadIdx.x];
    int64_t rl = r < rows ? r : rows - 1;
    if (KIND >= 2) {   // the row load waits for a 4-byte load of the same vector
        const uint32_t w0 = *reinterpret_cast<const uint32_t*>(src + rl * kVpr + c);
        fake_dep(rl, w0);
    }
    u32x4 v = __builtin_nontemporal_load(src + rl * kVpr + c);
    if (kBias) {
        if (threadIdx.x < 2 * SV) bl[threadIdx.x] = bq;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's LDS stores are done
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const float4 a0 = bl[2 * j], a1 = bl[2 * j + 1];
        const float bv[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        v = gelu8<true>(v, bv);
    } else {
        v.x ^= 0x3C003C00u;
    }
    if (r < rows) __builtin_nontemporal_store(v, dst + r * kVpr + c);
}

template <int WPR, int RPB, int KIND, int P>
int launch_slab(const void* s, void* d, const float* bias, int64_t rows, hipStream_t st) {
    const int64_t nb = (rows + RPB - 1) / RPB * (12 / WPR);
    const int64_t per = P == 0 ? nb : (nb + P - 1) / P;
    const dim3 grid = P == 0 ? dim3(12 / WPR, (unsigned)((rows + RPB - 1) / RPB)) : dim3((unsigned)(per * P));
    hipLaunchKernelGGL((slab_probe<WPR, RPB, KIND, P>), grid, dim3(WPR * RPB * 64), 0, st,
                       static_cast<const u32x4*>(s), static_cast<u32x4*>(d), bias, rows, nb, per);
    return (int)hipGetLastError();
}

// Rows of 1536 f16 (3 KB, the width of LN / QK / the gated residual): the
// [rows, 6144] buffers read as [4 * rows, 1536], 192 vectors per row.
//   MODE 0  one wave per row, 3 vectors per lane, 8 rows per block (LN / QK shape)
//   MODE 1  3 waves per row, one vector per lane, 4 rows per block (12 waves)
//   MODE 2  4 waves on 4 rows of one 1 KB piece; consecutive blocks walk the 3 pieces
//   MODE 3  3 waves per row, one vector per lane, 2 rows per block (6 waves)
//   MODE 4  one wave per row, 3 vectors per lane, 4 rows per block
//   MODE 5  MODE 0 whose row loads wait for one dependent 4-byte load of the
//           row first (as the QK kernel's row loads wait for its coordinates)
//   MODE 6  MODE 0 whose row loads wait for a 4-byte load of one word every
//           wave reads (an L2 hit after the first: a delay, no prefetch)
//   MODE 7  MODE 0 with the 4-byte loads of MODE 5 issued but not waited for
//           (the prefetch without the delay)
//   MODE 8  MODE 0 whose row loads wait for a 4-byte load of a separate
//           16-byte-per-row array (the QK kernel's coordinates)
//   MODE 9  MODE 7 with a 4-byte load in each of the row's three 1 KB pieces
//   MODE 10 MODE 7 with the 4-byte load non-temporal
//   MODE 11 MODE 7 with the 4-byte load in the row's second 1 KB piece
//   MODE 12 MODE 0 with the row loads without the non-temporal bit
//   MODE 13 MODE 0 with the first 1 KB piece's load without the non-temporal bit
constexpr int kNarrowVpr = 192;
template <int MODE>
constexpr bool narrow_wave_row() { return MODE == 0 || MODE == 4 || MODE >= 5; }
template <int MODE>
constexpr int narrow_waves() { return MODE == 0 || MODE >= 5 ? 8 : MODE == 1 ? 12 : MODE == 3 ? 6 : 4; }
template <int MODE>
constexpr int narrow_rows() { return MODE == 0 || MODE >= 5 ? 8 : MODE == 3 ? 2 : 4; }



template <int MODE>
__global__ __launch_bounds__(narrow_waves<MODE>() * 64) void narrow_probe(const u32x4* __restrict__ src,
                                                                           u32x4* __restrict__ dst, int64_t rows) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t b = blockIdx.x;
    if (narrow_wave_row<MODE>()) {
        const int64_t r = b * narrow_rows<MODE>() + wave;
        int64_t rl = r < rows ? r : rows - 1;
        uint32_t w7 = 0;
        if (MODE == 5 || MODE == 7) {
            // a word of each of the row's first 64 vectors
            const uint32_t w0 = *reinterpret_cast<const uint32_t*>(src + rl * kNarrowVpr + lane);
            if (MODE == 5) fake_dep(rl, w0);
            else w7 = w0;   // consumed after the row loads
        } else if (MODE == 9) {
            const uint32_t* q = reinterpret_cast<const uint32_t*>(src + rl * kNarrowVpr + lane);
            w7 = q[0] ^ q[256] ^ q[512];
        } else if (MODE == 10) {
            w7 = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src + rl * kNarrowVpr + lane));
        } else if (MODE == 11) {
            w7 = *reinterpret_cast<const uint32_t*>(src + rl * kNarrowVpr + 64 + lane);
        } else if (MODE == 6) {
            const uint32_t w0 = *reinterpret_cast<const uint32_t*>(src + lane);
            fake_dep(rl, w0);
        } else if (MODE == 8) {
            // 16 bytes per row in the last 16 * rows bytes of the destination
            // (written by the row stores only after this read, and rewritten by
            // them: the probe's output is not checked)
            const uint32_t w0 = *reinterpret_cast<const uint32_t*>(dst + (rows * kNarrowVpr - rows) + rl);
            fake_dep(rl, w0);
        }
        u32x4 v[3];
        const u32x4* q = src + rl * kNarrowVpr + lane;
        if constexpr (MODE == 12) {
            v[0] = q[0];
            v[1] = q[64];
            v[2] = q[128];
        } else if constexpr (MODE == 13) {
            v[0] = q[0];
            v[1] = __builtin_nontemporal_load(q + 64);
            v[2] = __builtin_nontemporal_load(q + 128);
        } else {
#pragma unroll
            for (int j = 0; j < 3; ++j) v[j] = __builtin_nontemporal_load(q + j * 64);
        }
        // MODE 7, 9-11: the lead word is waited for with the row loads, not before them
        if (MODE == 7 || (MODE >= 9 && MODE <= 11))
            asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]) : "v"(w7));
        if (r < rows) {
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                v[j].x ^= 0x3C003C00u;
                __builtin_nontemporal_store(v[j], dst + r * kNarrowVpr + j * 64 + lane);
            }
        }
    } else {
        int64_t r;
        int piece;
        if (MODE == 2) {
            piece = (int)(b % 3);
            r = b / 3 * 4 + wave;
        } else {
            piece = wave % 3;
            r = b * narrow_rows<MODE>() + wave / 3;
        }
        const int64_t rl = r < rows ? r : rows - 1;
        u32x4 v = __builtin_nontemporal_load(src + rl * kNarrowVpr + piece * 64 + lane);
        v.x ^= 0x3C003C00u;
        if (r < rows) __builtin_nontemporal_store(v, dst + r * kNarrowVpr + piece * 64 + lane);
    }
}

template <int MODE>
int launch_narrow(const void* s, void* d, const float*, int64_t rows, hipStream_t st) {
    const int64_t nrows = rows * 4;   // [rows, 6144] as [4 * rows, 1536]
    const int64_t nb = MODE == 2 ? (nrows + 3) / 4 * 3 : (nrows + narrow_rows<MODE>() - 1) / narrow_rows<MODE>();
    hipLaunchKernelGGL((narrow_probe<MODE>), dim3((unsigned)nb), dim3(narrow_waves<MODE>() * 64), 0, st,
                       static_cast<const u32x4*>(s), static_cast<u32x4*>(d), nrows);
    return (int)hipGetLastError();
}

// LayerNorm + modulate over rows of 1536 f16 with one 16-byte vector per
// lane: 3 waves per row, RPB rows per block. Each wave reduces its 512
// values to (sum, sum of squares about its own mean); the block's waves swap
// those through LDS behind one barrier (which also covers the staging of
// the shift and scale rows, f32 [2][1536] from `par`), and each combines its
// row's three pairs (Chan et al.'s pairwise update) into the row's mean and
// variance.
__device__ __forceinline__ float probe_wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

template <int RPB>
__global__ __launch_bounds__(RPB * 192) void lnrow_probe(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                         const float* __restrict__ par, int64_t rows) {
    __shared__ float4 ps[768];
    __shared__ float2 part[RPB * 3];
    const int wave = (int)(threadIdx.x >> 6);
    const int lane = (int)(threadIdx.x & 63);
    const int64_t r = (int64_t)blockIdx.x * RPB + wave / 3;
    const int piece = wave % 3;
    const int64_t rl = r < rows ? r : rows - 1;
    const u32x4 w = __builtin_nontemporal_load(src + rl * kNarrowVpr + piece * 64 + lane);
    for (int i = (int)threadIdx.x; i < 768; i += RPB * 192) ps[i] = reinterpret_cast<const float4*>(par)[i];
    const uint32_t in[4] = {w.x, w.y, w.z, w.w};
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(in[i] & 0xFFFFu));
        x[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(in[i] >> 16));
    }
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) sum += x[i];
    sum = probe_wave_sum(sum);
    const float mw = sum * (1.0f / 512.0f);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) q += (x[i] - mw) * (x[i] - mw);
    q = probe_wave_sum(q);
    if (lane == 0) part[wave] = make_float2(sum, q);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (r >= rows) return;
    const int w0 = wave / 3 * 3;
    const float2 p0 = part[w0], p1 = part[w0 + 1], p2 = part[w0 + 2];
    const float mean = (p0.x + p1.x + p2.x) * (1.0f / 1536.0f);
    const float d0 = p0.x * (1.0f / 512.0f) - mean, d1 = p1.x * (1.0f / 512.0f) - mean,
                d2 = p2.x * (1.0f / 512.0f) - mean;
    const float m2 = p0.y + p1.y + p2.y + 512.0f * (d0 * d0 + d1 * d1 + d2 * d2);
    const float inv = __builtin_amdgcn_rsqf(m2 * (1.0f / 1536.0f) + 1e-6f);
    const int c4 = (piece * 512 + lane * 8) / 4;
    const float4 sh0 = ps[c4], sh1 = ps[c4 + 1], sc0 = ps[384 + c4], sc1 = ps[384 + c4 + 1];
    const float sh[8] = {sh0.x, sh0.y, sh0.z, sh0.w, sh1.x, sh1.y, sh1.z, sh1.w};
    const float sc[8] = {sc0.x, sc0.y, sc0.z, sc0.w, sc1.x, sc1.y, sc1.z, sc1.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = (x[2 * i] - mean) * inv * (1.0f + sc[2 * i]) + sh[2 * i];
        const float hi = (x[2 * i + 1] - mean) * inv * (1.0f + sc[2 * i + 1]) + sh[2 * i + 1];
        o[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
    }
    __builtin_nontemporal_store((u32x4){o[0], o[1], o[2], o[3]}, dst + r * kNarrowVpr + piece * 64 + lane);
}

template <int RPB>
int launch_lnrow(const void* s, void* d, const float* par, int64_t rows, hipStream_t st) {
    const int64_t nrows = rows * 4;   // [rows, 6144] as [4 * rows, 1536]
    hipLaunchKernelGGL((lnrow_probe<RPB>), dim3((unsigned)((nrows + RPB - 1) / RPB)), dim3(RPB * 192), 0, st,
                       static_cast<const u32x4*>(s), static_cast<u32x4*>(d), par, nrows);
    return (int)hipGetLastError();
}

// Cache-policy bits of the 16-byte loads and stores, in the slab copy shape
// (one vector per thread, 4 rows of one 1 KB column piece per block, 2-D
// grid). Buffer instructions carry the bits as an immediate: bit 0 sc0,
// bit 1 nt, bit 4 sc1. Each block's buffer descriptors start at its first
// row and span its rows, so the 32-bit offsets stay small.
template <int LA, int SA>
__global__ __launch_bounds__(256) void policy_probe(void* src, void* dst, int64_t rows) {
    constexpr int64_t kRowBytes = (int64_t)kVpr * 16;
    const int64_t r0 = (int64_t)blockIdx.y * 4;
    const int w = (int)(threadIdx.x >> 6);
    const int nr = (int)(rows - r0 < 4 ? rows - r0 : 4);
    const int wl = w < nr ? w : nr - 1;
    const int c = (int)blockIdx.x * 64 + (int)(threadIdx.x & 63);
    const int bytes = nr * (int)kRowBytes;
    const __amdgpu_buffer_rsrc_t s =
        __builtin_amdgcn_make_buffer_rsrc(static_cast<char*>(src) + r0 * kRowBytes, 0, bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t d =
        __builtin_amdgcn_make_buffer_rsrc(static_cast<char*>(dst) + r0 * kRowBytes, 0, bytes, 0x00020000);
    u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(s, (wl * kVpr + c) * 16, 0, LA);
    v.x ^= 0x3C003C00u;
    if (w < nr) __builtin_amdgcn_raw_buffer_store_b128(v, d, (w * kVpr + c) * 16, 0, SA);
}

template <int LA, int SA>
int launch_policy(const void* s, void* d, const float*, int64_t rows, hipStream_t st) {
    hipLaunchKernelGGL((policy_probe<LA, SA>), dim3(kVpr / 64, (unsigned)((rows + 3) / 4)), dim3(256), 0, st,
                       const_cast<void*>(s), d, rows);
    return (int)hipGetLastError();
}

// The same probe writing its output over its input (each thread stores
// exactly the vectors it loaded).
template <Launch F>
int in_place(const void* s, void*, const float* bias, int64_t rows, hipStream_t st) {
    return F(s, const_cast<void*>(s), bias, rows, st);
}

struct Probe {
    const char* name;
    Launch fn;
};
const Probe kProbes[] = {
    {"copy rpt1 P1", launch<768, 1, 0, 1>},      {"copy rpt1 P8", launch<768, 1, 0, 8>},
    {"copy rpt4 P1", launch<768, 4, 0, 1>},      {"copy rpt4 P8", launch<768, 4, 0, 8>},
    {"gelu rpt1 P8", launch<768, 1, 2, 8>},      {"gelu rpt4 P1", launch<768, 4, 2, 1>},
    {"gelu+bias rpt1 P8", launch<768, 1, 1, 8>}, {"gelu+bias rpt2 P2", launch<768, 2, 1, 2>},
    {"gelu+bias rpt4 P1", launch<768, 4, 1, 1>}, {"gelu+bias rpt4 P8", launch<768, 4, 1, 8>},
    // rows per thread against block width, and the order of a thread's rows
    {"copy W256 rpt1 P1", launch<256, 1, 0, 1>}, {"copy W256 rpt2 P1", launch<256, 2, 0, 1>},
    {"copy W256 rpt3 P1", launch<256, 3, 0, 1>}, {"copy W256 rpt4 P1", launch<256, 4, 0, 1>},
    {"copy W128 rpt6 P1", launch<128, 6, 0, 1>}, {"copy rpt4 P1 serial", launch<768, 4, 0, 1, 1>},
    {"copy rpt4 P1 strided", launch<768, 4, 0, 1, 0, 1>},
    {"gelu+bias W384 rpt2 P1", launch<384, 2, 1, 1>}, {"gelu+bias W256 rpt3 P1", launch<256, 3, 1, 1>},
    // the attention pack's head-major fan-out
    {"slab copy row-major", launch_hm<0>}, {"slab copy head-major direct", launch_hm<1>},
    {"slab copy head-major via LDS", launch_hm<2>},
    // in place: the stores go to the lines the loads just read
    {"copy W256 rpt1 P1 in place", in_place<launch<256, 1, 0, 1>>},
    {"copy rpt4 P1 in place", in_place<launch<768, 4, 0, 1>>},
    {"gelu+bias rpt4 P1 in place", in_place<launch<768, 4, 1, 1>>},
    {"slab copy row-major in place", in_place<launch_hm<0>>},
    {"piece-order copy row-major", launch_hm<3>}, {"piece-order copy head-major direct", launch_hm<4>},
    // one row per thread, rows of a block sharing the bias through LDS
    {"slab copy 1x8", launch_slab<1, 8, 0, 1>},   {"slab copy 1x4", launch_slab<1, 4, 0, 1>},
    {"slab copy 2x4", launch_slab<2, 4, 0, 1>},   {"slab copy 4x4", launch_slab<4, 4, 0, 1>},
    {"slab copy 4x2", launch_slab<4, 2, 0, 1>},   {"slab copy 1x16", launch_slab<1, 16, 0, 1>},
    {"slab copy 1x8 P8", launch_slab<1, 8, 0, 8>}, {"slab copy 4x4 P8", launch_slab<4, 4, 0, 8>},
    {"slab gelu+bias 1x8", launch_slab<1, 8, 1, 1>},   {"slab gelu+bias 1x4", launch_slab<1, 4, 1, 1>},
    {"slab gelu+bias 2x4", launch_slab<2, 4, 1, 1>},   {"slab gelu+bias 4x4", launch_slab<4, 4, 1, 1>},
    {"slab gelu+bias 4x2", launch_slab<4, 2, 1, 1>},   {"slab gelu+bias 1x16", launch_slab<1, 16, 1, 1>},
    {"slab gelu+bias 1x8 P8", launch_slab<1, 8, 1, 8>}, {"slab gelu+bias 4x4 P8", launch_slab<4, 4, 1, 8>},
    {"slab gelu+bias 1x4 2-D grid", launch_slab<1, 4, 1, 0>}, {"slab gelu+bias 1x2", launch_slab<1, 2, 1, 1>},
    {"slab copy 1x4 2-D grid", launch_slab<1, 4, 0, 0>},
    {"slab copy 1x4 2-D grid lead load", launch_slab<1, 4, 2, 0>},
    {"slab gelu+bias 1x4 2-D grid lead load", launch_slab<1, 4, 3, 0>},
    // 3 KB rows (1536 f16)
    {"narrow copy wave per row x8", launch_narrow<0>}, {"narrow copy wave per row x4", launch_narrow<4>},
    {"narrow copy 3 waves per row x4", launch_narrow<1>}, {"narrow copy 3 waves per row x2", launch_narrow<3>},
    {"narrow copy 1 KB piece x4 rows", launch_narrow<2>},
    {"narrow copy wave per row x8 dependent lead load", launch_narrow<5>},
    {"narrow copy wave per row x8 shared lead load", launch_narrow<6>},
    {"narrow copy wave per row x8 lead load no wait", launch_narrow<7>},
    {"narrow copy wave per row x8 side-array lead load", launch_narrow<8>},
    {"narrow copy wave per row x8 lead load per piece", launch_narrow<9>},
    {"narrow copy wave per row x8 nt lead load", launch_narrow<10>},
    {"narrow copy wave per row x8 lead load second piece", launch_narrow<11>},
    {"narrow copy wave per row x8 cached row loads", launch_narrow<12>},
    {"narrow copy wave per row x8 first piece cached", launch_narrow<13>},
    {"narrow LN+modulate 3 waves per row x4", launch_lnrow<4>},
    {"narrow LN+modulate 3 waves per row x2", launch_lnrow<2>},
    {"narrow LN+modulate 3 waves per row x1", launch_lnrow<1>},
    // cache-policy bits (load / store): 0 none, 2 nt, 16 sc1, 17 sc0 sc1, 18 nt sc1
    {"policy copy L nt S nt", launch_policy<2, 2>},   {"policy copy L - S -", launch_policy<0, 0>},
    {"policy copy L - S nt", launch_policy<0, 2>},    {"policy copy L nt S -", launch_policy<2, 0>},
    {"policy copy L nt S nt sc1", launch_policy<2, 18>}, {"policy copy L nt S sc0 sc1", launch_policy<2, 17>},
    {"policy copy L nt sc1 S nt", launch_policy<18, 2>}, {"policy copy L sc1 S sc1", launch_policy<16, 16>},
};

}  // namespace

extern "C" int hbm_probe_count() { return (int)(sizeof(kProbes) / sizeof(kProbes[0])); }
extern "C" const char* hbm_probe_name(int i) {
    return (i >= 0 && i < hbm_probe_count()) ? kProbes[i].name : "";
}
// src, dst: f16 [rows, 6144] (16-byte aligned); bias: f32 [6144].
extern "C" int hbm_probe_launch(int i, const void* src, void* dst, const float* bias, int64_t rows, void* stream) {
    if (i < 0 || i >= hbm_probe_count() || rows <= 0) return -1;
    return kProbes[i].fn(src, dst, bias, rows, static_cast<hipStream_t>(stream));
}
