// The qkv linear fused with the self-attention epilogue and the head-major
// pack (t2h_qkv_linear_pack), on the GEMM core (tiling and pipeline:
// t2h_gemm_core.h): a wave's 128 features are one head of 128 or two heads of
// 64. T2H_QKV_WAVES picks
// the layout: 8 (shipped; 64 tokens per wave, 128 accumulators, 10 % faster
// on the config-5 qkv) or 4 (128 tokens per wave, direct-to-LDS loads).
//
// Reference: the qkv enqueue_gemm + bias_rms_rope_qkv + pack_q_z + pack_kv_z
// of the self-attention chain (gpu/attention.mojo:507-563, 566-594, 634-662,
// sequence 983-1013).
#ifndef T2H_QKV_WAVES
#define T2H_QKV_WAVES 8
#endif
#define T2H_GEMM_WAVES T2H_QKV_WAVES
#include "t2h_gemm_core.h"

namespace t2h {
namespace {

// ---- qkv linear + attention epilogue + head-major pack ----------------------
// The qkv GEMM's output [rows, 3, H, HD] never reaches memory. A wave's 128
// features are one head of HD = 128 or two heads of HD = 64 (q, k or v: head
// hg = n / HD, tensor hg / H, head hg % H) for kWT tokens (64 with 8 waves,
// 128 with 4), and each token's head lives in two lanes (l and l ^ 32, 64 or
// 32 values each: the MFMA tile of feature tile fi holds features fi*32 +
// 8q + 4h + i in lane half h). Per token, in the
// order of the separate kernels
// (bias_rms_rope_qkv, pack_q_z, pack_kv_z): + bias; q/k: RMS over the head,
// x * rsqrt(sum x^2) * (gamma * sqrt(D)); q/k: RoPE on the in-lane pairs
// (2p, 2p + 1) with cos/sin from the phase table or from the token's
// position; q: * 1/sqrt(D); tokens >= rows: 0. The head then goes through
// the wave's own LDS region (kStaged tokens at a time: 64 with 4 waves, 32
// with 8, 16 KB or 8 KB) as 256-byte token rows (one or two heads) and
// leaves as 16-byte vectors: whole token rows of each head (qh [H, mp, D],
// k [H, lp, D], vh [H, lp, D]) or, for the transposed k [H, D, lp], 8 tokens
// of one feature gathered from 8 rows. Tiles past the last token row skip the
// GEMM and write the pads.
constexpr int kHead = 128;   // features of a wave (one staged token row: 256 bytes of 16-bit values)
static_assert(kTJ == 2 || kTJ == 4, "copy_col cases");
constexpr int kStaged = kWaves == 8 ? 32 : 64;   // token rows a wave stages at a time
constexpr int kJJ = kStaged / 32;                // token tiles per staged group
constexpr int kRegion = kStaged * 256;           // bytes of a wave's staging region
constexpr int kParamOff = kWaves * kRegion;      // [head][bias, gamma * sqrt(D)][128] f32
constexpr int kPPT = 2 * 2 * kHead / kGemmThreads;   // parameters per thread
// 8 waves unroll their two groups, so that each group's accumulators are used
// in place and are dead after it (128 accumulators in 256 registers); 4 waves
// keep the loop (a runtime token tile picks its accumulators by a switch).
constexpr int kGrpUnroll = kWaves == 8 ? kTJ / kJJ : 1;

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

template <typename T, bool KT, int HD>
__global__ __launch_bounds__(kGemmThreads, T2H_GEMM_OCC) void qkv_pack_kernel(GemmArgs g, PackArgs p, RopeSlots tab) {
    constexpr int NH = kHead / HD;    // heads per wave
    constexpr int FPH = kFI / NH;     // 32-feature MFMA tiles per head
    constexpr int CPH = HD / 8;       // 16-byte chunks of a head's token row
    // One LDS array: the GEMM's stages, then the epilogue's staging (a
    // region per wave) and the tile's parameters at 64 KB. (A separate
    // parameter array that took the kernel past 128 KB of LDS measured 20 %
    // slower on MI355X.)
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];
    static_assert(kWF == kHead && kHead % HD == 0 && kFI % NH == 0 && kWT % kStaged == 0 &&
                      kParamOff + 2 * 2 * kHead * 4 <= kStages * kStageBytes,
                  "staging layout");
    static_assert(kPPT * kGemmThreads == 2 * 2 * kHead, "parameters per thread");
    TileOf tile;
    if (!tile.init(g)) return;
    const int64_t t0 = tile.t0, n0 = tile.n0;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wf = wave & 1, wt = wave >> 1;
    const int fr = lane & 31, h = lane >> 5;
    const int hg = (int)((n0 + wf * kWF) / HD);
    const int which = hg / p.heads;          // 0 q, 1 k, 2 v (the wave's heads share it: 128 | H * HD)
    const int z = hg - which * p.heads;      // the wave's first head
    const float* __restrict__ bias = which == 0 ? p.bias_q : which == 1 ? p.bias_k : p.bias_v;
    const float* __restrict__ gamma = which == 0 ? p.gamma_q : which == 1 ? p.gamma_k : nullptr;

    // the tile's bias and gamma * sqrt(D) (slot i = (wave group * 2 + kind) *
    // 128 + d, kPPT slots per thread; a group's 128 features are consecutive
    // in the [H * HD] parameter rows) are requested before the GEMM and land
    // in LDS after it
    float pv[kPPT];
#pragma unroll
    for (int j = 0; j < kPPT; ++j) {
        const int i = (int)threadIdx.x + j * kGemmThreads;
        const int ph = i / (2 * kHead), kind = (i / kHead) & 1, pd = i % kHead;
        const int hp = (int)((n0 + ph * kWF) / HD);
        const int wp = hp / p.heads;
        const int pz = hp - wp * p.heads;
        const float* src = kind == 0 ? (wp == 0 ? p.bias_q : wp == 1 ? p.bias_k : p.bias_v)
                                     : (wp == 0 ? p.gamma_q : wp == 1 ? p.gamma_k : nullptr);
        pv[j] = src != nullptr ? src[pz * HD + pd] : 0.0f;
    }
    f32x16 acc[kFI][kTJ];
    zero_acc(acc);
    if (t0 < g.rows) gemm_mainloop<T>(g, t0, n0, lds, acc);   // block-uniform (ends with a barrier)
    float* prm = reinterpret_cast<float*>(lds + kParamOff);
#pragma unroll
    for (int j = 0; j < kPPT; ++j) {
        const int i = (int)threadIdx.x + j * kGemmThreads;
        prm[i] = ((i / kHead) & 1) ? pv[j] * p.rms_scale : pv[j];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();

    const bool rope = p.use_rope && which < 2 && g.rows > 0;
    const int64_t extent = which == 0 ? p.mp : p.lp;
    T* __restrict__ out = static_cast<T*>(which == 0 ? p.qh : which == 1 ? p.k_out : p.vh);
    const bool trans = KT && which == 1;
    uint8_t* region = lds + wave * kRegion;
    const float* pb = prm + (wf * 2 + 0) * kHead;
    const float* pg = prm + (wf * 2 + 1) * kHead;

#pragma unroll kGrpUnroll
    for (int grp = 0; grp < kTJ / kJJ; ++grp) {
#pragma unroll kGrpUnroll
        for (int jj = 0; jj < kJJ; ++jj) {
            const int tj = grp * kJJ + jj;
            // this token tile's accumulators (static register indices per case)
            float col[kFI][16];
            switch (tj) {
                case 0: copy_col<0>(acc, col); break;
                case 1: copy_col<1>(acc, col); break;
                case 2: copy_col<(kTJ > 2 ? 2 : 0)>(acc, col); break;
                default: copy_col<(kTJ > 2 ? 3 : 1)>(acc, col); break;
            }
            const int tl = jj * 32 + fr;                      // staged row (token within the group)
            const int64_t t = t0 + wt * kWT + tj * 32 + fr;
            const int64_t tc = t < g.rows ? t : g.rows - 1;   // clamped for position reads
            const bool live = t < g.rows;
            // feature of col[fi][4q + i]: d = fi*32 + 8q + 4h + i
            // the token's cos/sin (table path) are requested first and arrive
            // while the bias and the sum of squares are computed
            float cs[kFI][4][4];
            const bool table = rope && p.phases != nullptr;
            if (table) {
                const float* row = p.phases + (tc % p.phase_rows) * HD;
#pragma unroll
                for (int fi = 0; fi < kFI; ++fi)
#pragma unroll
                    for (int q = 0; q < 4; ++q) load_params<4>(row + (fi % FPH) * 32 + q * 8 + h * 4, cs[fi][q]);
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
            // each head's sum of squares: HD / 2 values here, HD / 2 in lane ^ 32
            float rn[NH];
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) rn[hh] = 1.0f;
            if (gamma != nullptr) {
#pragma unroll
                for (int hh = 0; hh < NH; ++hh) {
                    float ss = 0.0f;
#pragma unroll
                    for (int fi = hh * FPH; fi < (hh + 1) * FPH; ++fi) ss += sum_sq<16>(col[fi]);
                    ss += __shfl_xor(ss, 32);
                    rn[hh] = ss < 1e-24f ? 1e12f : __builtin_amdgcn_rsqf(ss);
                }
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
                        const float r = rn[fi / FPH];
                        v[q * 4 + 0] = (v[q * 4 + 0] * r) * g4.x;
                        v[q * 4 + 1] = (v[q * 4 + 1] * r) * g4.y;
                        v[q * 4 + 2] = (v[q * 4 + 2] * r) * g4.z;
                        v[q * 4 + 3] = (v[q * 4 + 3] * r) * g4.w;
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
                                const int sl = ((fi % FPH) * 32 + q * 8 + h * 4) / 2 + j;
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
        const int64_t tw = t0 + wt * kWT + grp * kStaged;   // first token of the staged rows
        if (!trans) {
            // token rows: 16 lanes per 256-byte row, 4 rows per instruction
#pragma unroll 4
            for (int it = 0; it < kStaged / 4; ++it) {
                const int row = it * 4 + (lane >> 4);
                const int c = lane & 15;
                const u32x4 w = *reinterpret_cast<const u32x4*>(region + row * 256 + ((c ^ stage_swz(row)) * 16));
                const int64_t t = tw + row;
                if (t < extent) out_store16(out + ((int64_t)(z + c / CPH) * extent + t) * HD + (c % CPH) * 8, w);
            }
        } else {
            // feature rows of the transposed k: lane (d, g) gathers feature d
            // of tokens 8g .. 8g + 7 (eight 2-byte reads, one per token row);
            // kG groups of 8 tokens, 64 / kG features per instruction
            constexpr int kG = kStaged / 8;
#pragma unroll 2
            for (int it = 0; it < kHead * kG / 64; ++it) {
                const int d = it * (64 / kG) + lane / kG;
                const int gg = lane % kG;
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
                    out_store16(out + ((int64_t)z * HD + d) * p.lp + t, w);
                }
            }
        }
        // the next group overwrites the staged rows: every lane's reads are done
        __builtin_amdgcn_s_waitcnt(0xC07F);
    }
}

template <typename T, int HD>
hipError_t qkv_typed(const GemmArgs& g, const PackArgs& p, const RopeSlots& tab, hipStream_t s) {
    const dim3 grid = grid_1d(g.nblocks), blk(kGemmThreads);
    if (p.k_transposed) hipLaunchKernelGGL((qkv_pack_kernel<T, true, HD>), grid, blk, 0, s, g, p, tab);
    else hipLaunchKernelGGL((qkv_pack_kernel<T, false, HD>), grid, blk, 0, s, g, p, tab);
    return hipGetLastError();
}

}  // namespace

bool gemm_head_dim_ok(int32_t head_dim) { return head_dim == 128 || head_dim == 64; }

hipError_t launch_qkv_pack(GemmArgs g, const PackArgs& p, const RopeSlots& tab, hipStream_t s) {
    // token tiles cover the pad rows of the outputs too (they are written as 0)
    int64_t span = g.rows;
    if (p.mp > span) span = p.mp;
    if (p.lp > span) span = p.lp;
    g.ftiles = g.n / kBF;
    g.nblocks = ((span + kBT - 1) / kBT) * g.ftiles;
    g.tgroup = tile_group(g.k);
    if (g.nblocks == 0) return hipSuccess;
    if (p.head_dim == 64) {
        if (g.dtype == T2H_F16) return qkv_typed<_Float16, 64>(g, p, tab, s);
        return qkv_typed<__bf16, 64>(g, p, tab, s);
    }
    if (g.dtype == T2H_F16) return qkv_typed<_Float16, 128>(g, p, tab, s);
    return qkv_typed<__bf16, 128>(g, p, tab, s);
}

}  // namespace t2h
