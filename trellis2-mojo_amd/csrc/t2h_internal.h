// Launcher interface between the C-ABI layer (t2h_api.hip) and the kernel
// translation units. Arguments arrive validated; launchers only pick a kernel
// instantiation and a grid, then enqueue.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "t2h.h"

#ifndef T2H_FRONTS
#define T2H_FRONTS 1   // block order over contiguous fronts (front_of in t2h_device.h)
#endif

namespace t2h {

struct BatchArgs {
    const int64_t* offsets;
    int32_t nbatch;
    int64_t rows_per_batch;
};

struct LnArgs {
    const void* x;       // [rows, cols]
    const void* h;       // residual branch (fused join) or nullptr
    void* x_out;         // fused join: updated residual stream
    void* y_out;         // normalised (+ epilogue) output
    const float* bias;   // join: h bias [cols] or nullptr
    const float* gate;   // join: gate rows or nullptr
    int64_t gate_stride;
    float eps;
    int32_t mode;        // T2H_LN_*
    const float* p0;
    const float* p1;
    int64_t p_stride;
    int64_t rows;
    int32_t cols;
    int32_t dtype;
    BatchArgs batch;
    int64_t fper;        // logical blocks per front (set at launch)
    int32_t cached;      // fast path: first row piece with the cached policy (set at launch)
};

// Per-slot RoPE table, passed by value as a kernel argument: slot p rotates
// pair (2p, 2p+1) by angle pos[axis[p]] * freq[p]; axis -1 = identity slot.
struct RopeSlots {
    float freq[T2H_MAX_HALF_HEAD];
    int8_t axis[T2H_MAX_HALF_HEAD];
};

struct QkArgs {
    const void* q_in;
    const void* k_in;
    void* q_out;
    void* k_out;
    void* v;                 // packed-qkv v (bias only) or nullptr
    int64_t rows;
    int64_t in_stride;
    int64_t out_stride;
    int32_t heads;
    int32_t head_dim;
    int32_t dtype;
    const float* bias_q;
    const float* bias_k;
    const float* bias_v;
    const float* gamma_q;    // nullptr = no RMS
    const float* gamma_k;
    float rms_scale;         // f32(sqrt(f64(head_dim)))
    int32_t use_rope;
    int32_t pos_dim;
    int32_t freq_dim;        // distinct rotary frequencies (slot p uses freq p % freq_dim)
    const float* phases;     // position source 1
    int64_t phase_rows;
    const int32_t* coords;   // position source 2
    int32_t coord_cols;
    int32_t grid_res;        // position source 3
    int64_t fper;            // logical tiles per front (set at launch)
};

// Self-attention epilogue + head-major packing (t2h_attn_pack).
struct PackArgs {
    const void* q;           // [rows, H, D] rows in_stride apart; any may be nullptr
    const void* k;
    const void* v;
    int64_t rows;
    int64_t in_stride;
    int32_t heads;
    int32_t head_dim;
    int32_t dtype;
    const float* bias_q;
    const float* bias_k;
    const float* bias_v;
    const float* gamma_q;    // nullptr = no RMS
    const float* gamma_k;
    float rms_scale;         // f32 sqrt(head_dim)
    float q_scale;           // 1 / f32 sqrt(head_dim), baked into qh
    int32_t use_rope;
    int32_t pos_dim;
    const float* phases;
    int64_t phase_rows;
    const int32_t* coords;
    int32_t coord_cols;
    int32_t grid_res;
    void* qh;                // [H, mp, D]
    int64_t mp;
    void* k_out;             // [H, D, lp] (k_transposed) or [H, lp, D]
    void* vh;                // [H, lp, D]
    int64_t lp;
    int32_t k_transposed;
};

// Weight GEMM on MFMA (t2h_linear, t2h_qkv_linear_pack):
// acc[t, n] = sum_k x[t, k] * w[n, k], f16/bf16 operands, f32 accumulation,
// then an epilogue in the store (bias + activation, or the attention pack).
struct GemmArgs {
    const void* x;           // [rows, k], rows ldx elements apart
    int64_t ldx;
    const void* w;           // [n, k] contiguous (a linear's [out, in] weight)
    int64_t rows;
    int32_t n;               // output features, a multiple of the feature tile
    int32_t k;               // input features, a multiple of the k step
    int32_t dtype;           // operand storage: T2H_F16 / T2H_BF16
    const float* bias;       // [n] f32 or nullptr
    int32_t act;             // T2H_ACT_* or -1 (none)
    void* out;               // [rows, n], rows ldo elements apart
    int64_t ldo;
    int32_t out_dtype;       // T2H_F32 or dtype
    int64_t nblocks;         // set by the launcher: token tiles x feature tiles
    int32_t ftiles;          // feature tiles
    int32_t tgroup;          // set by the launcher: token tiles per group of the tile order
    // residual epilogue (t2h_linear_gate_residual): out = res + fl(fl(acc + bias) * gate[b])
    const void* res;         // [rows, n], rows ldo elements apart, out_dtype; may alias out
    const float* gate;       // gate rows [nbatch, n] gate_stride apart, or nullptr (ungated)
    int64_t gate_stride;
    BatchArgs batch;
};

// Flow-matching Euler step (t2h_flow_euler_step).
constexpr int kEulerBlock = 256;          // threads per block of the elementwise pass
#ifndef T2H_EULER_CHUNK
#define T2H_EULER_CHUNK 2048
#endif
#ifndef T2H_EULER_VEC
#define T2H_EULER_VEC 1   // 0: the scalar path for every call (tuning comparisons)
#endif
#ifndef T2H_STATS_PER
#define T2H_STATS_PER 16
#endif
constexpr int kEulerChunk = T2H_EULER_CHUNK;   // elements per block of the elementwise pass
#ifndef T2H_STATS_BLOCK
#define T2H_STATS_BLOCK 1024
#endif
#ifndef T2H_STATS_MAXSEG
#define T2H_STATS_MAXSEG 256
#endif
#ifndef T2H_STATS_MINSHARE
#define T2H_STATS_MINSHARE 16384
#endif
constexpr int kStatsBlock = T2H_STATS_BLOCK;   // threads per block of the rescale's statistics pass
constexpr int kStatsPer = T2H_STATS_PER;  // elements per thread per tensor in one statistics load group
constexpr int kStatsChunk = kStatsBlock * kStatsPer;   // elements of one load group of a block
constexpr int kStatsMaxPerSeg = T2H_STATS_MAXSEG;   // statistics blocks (f64 partials) per segment, at most
constexpr int kStatsMinShare = T2H_STATS_MINSHARE;  // a segment gets one statistics block per this many elements
constexpr int kEulerMaxSeg = 64;          // varlen segments carried in the kernel arguments
// statistics blocks the built-in scratch of t2h_flow_euler_step_noalloc holds:
// every split into kEulerMaxSeg segments at the per-segment cap
// (16,384 f64 quads = 512 KB per GPU)
constexpr int kEulerScratchPartials = kEulerMaxSeg * kStatsMaxPerSeg;
// a block of the elementwise pass covers whole 16-byte vectors of every
// storage type on every thread (8 elements of 16-bit storage)
static_assert(kEulerChunk % (kEulerBlock * 8) == 0, "T2H_EULER_CHUNK: a multiple of 8 * kEulerBlock");
static_assert(kStatsPer % 8 == 0, "T2H_STATS_PER: whole 16-byte vectors of every storage type");
static_assert(kStatsBlock % 64 == 0 && kStatsBlock <= 1024, "T2H_STATS_BLOCK: whole waves, one block");
// One-launch rescale (a single segment whose three tensors fit in the
// registers of one resident grid): the workspace starts with the grid
// barrier's words (kEulerBarBytes: an error word, 8 release slots of 128
// bytes, and per block a 64-bit arrival flag, a leave mark and a claim
// word), then one f64 partial quad per block.
constexpr int kFuseBlock = 256;           // threads per block
constexpr int kFuseMaxBlocks = 2048;      // blocks (partials) the workspace is sized for: the most
                                          // 256-thread blocks 256 CUs hold at once (8 per CU)
constexpr int kEulerBarBytes = 64 + 8 * 128 + 3 * kFuseMaxBlocks * 8;
constexpr int64_t kFuseBytes = kEulerBarBytes + (int64_t)kFuseMaxBlocks * 32;
static_assert(kFuseBytes <= (int64_t)kEulerScratchPartials * 32, "the built-in scratch holds the one-launch form");
struct EulerArgs {
    const void* x;
    const void* v_pos;
    const void* v_neg;
    void* x_prev;
    void* pred_x0;           // nullptr = not written
    int64_t n;               // elements
    int64_t row_size;
    int32_t dtype;
    int32_t mode;            // 0: pred = v_pos, 1: CFG combine, 2: CFG + rescale
    float gp, gn;            // f32(g), f32(1 - g)
    float a, cc, dt;         // f32(1 - sigma_min), f32(sigma_min + (1 - sigma_min) t), f32(t - t_prev)
    float gr, one_m_gr;      // f32(guidance_rescale), 1 - that (in f32)
    int32_t vec;             // 1: every tensor 16-byte aligned and every block bound a multiple
                             //    of the 16-byte element count -> vector loads/stores
    int32_t uniform;         // 1: segment = row (dense), 0: bounds[] (varlen)
    int32_t nseg;
    int64_t bounds[kEulerMaxSeg + 1];    // element bounds of the varlen segments
    int64_t blk_base[kEulerMaxSeg + 1];  // first elementwise block of each varlen segment
    int64_t pbase[kEulerMaxSeg + 1];     // first statistics block (partial) of each varlen segment
    int32_t pper;            // statistics blocks per row (uniform)
    int64_t nblocks;         // blocks of the elementwise pass
    int64_t nstats;          // blocks of the statistics pass (= f64 partials)
    double* partial;         // [nstats][4] workspace: sum x0_pos, sum x0_pos^2, sum x0_cfg, sum x0_cfg^2
    // one-launch rescale: set by the host when the call may take it (one
    // segment [fuse_lo, fuse_hi) on whole vectors, a workspace of kFuseBytes);
    // the launcher takes it when the segment fits the resident grid
    int32_t fuse;
    int32_t fuse_polls;      // polls a data block waits for the ratio before it leaves its vectors
    int64_t fuse_lo, fuse_hi;
    void* fuse_ws;           // the workspace: barrier words, then the partial quads
};

struct PhaseArgs {
    float* out;
    int64_t rows;
    int32_t head_dim;
    int32_t pos_dim;
    const float* positions;
    const int32_t* coords;
    int32_t coord_cols;
    int32_t grid_res;
};

struct EltArgs {
    const void* x;
    const void* h;
    void* out;
    const float* bias;
    const float* gate;     // gate rows / modulate scale / binop other
    const float* shift;    // modulate shift
    int64_t p_stride;
    int64_t rows;
    int32_t cols;
    int32_t other_cols;    // binop: cols or 1
    int32_t dtype;
    int32_t kind;          // activation kind / binop op
    BatchArgs batch;
    int32_t col_tiles;     // row-tiled kernels: blocks across one row (set at launch)
    int64_t fper;          // logical blocks per front (set at launch)
    int32_t block_threads; // the launch's block width (set at launch): read from the
                           // arguments, since blockDim.x costs a vector load per wave
    int32_t cached;        // gated residual: a tile's first residual row cached (set at launch)
};

// Grid of nblocks blocks. A dispatch counts work-items in 32 bits per grid
// dimension, so past 2^20 blocks the grid becomes 2^20 x ceil(nblocks/2^20);
// kernels launched on it index blocks with block_linear() and return when it
// is past their last block.
constexpr int64_t kGridX = int64_t(1) << 20;
inline dim3 grid_1d(int64_t nblocks) {
    if (nblocks <= kGridX) return dim3((unsigned)nblocks);
    return dim3((unsigned)kGridX, (unsigned)((nblocks + kGridX - 1) / kGridX));
}
// Logical blocks per front and the physical block count of a launch in
// T2H_FRONTS fronts (front_of() in t2h_device.h); kernels return on logical
// blocks past their last one.
inline int64_t front_per(int64_t nblocks) { return (nblocks + T2H_FRONTS - 1) / T2H_FRONTS; }
inline int64_t front_grid(int64_t nblocks) { return front_per(nblocks) * T2H_FRONTS; }

// t2h_norm.hip
hipError_t launch_ln(const LnArgs& a, hipStream_t s);
// t2h_qk.hip
hipError_t launch_qk(const QkArgs& a, const RopeSlots& tab, hipStream_t s);
hipError_t launch_phases(const PhaseArgs& a, const RopeSlots& tab, hipStream_t s);
hipError_t launch_pack(const PackArgs& a, const RopeSlots& tab, hipStream_t s);
// t2h_gemm.hip
hipError_t launch_gemm(GemmArgs a, hipStream_t s);
int32_t gemm_feature_tile();   // output features per block (out_features must be a multiple)
int32_t gemm_k_step();         // k per stage (in_features must be a multiple)
bool gemm_head_dim_ok(int32_t head_dim);   // head_dim the fused qkv GEMM + pack takes (64, 128)
hipError_t launch_qkv_pack(GemmArgs g, const PackArgs& p, const RopeSlots& tab, hipStream_t s);
hipError_t launch_gemm_residual(GemmArgs a, hipStream_t s);
// t2h_sampler.hip
hipError_t launch_euler(const EulerArgs& a, int64_t cover_lo, int64_t cover_hi, hipStream_t s);
// Device address of the current device's built-in statistics scratch
// (kEulerScratchPartials f64 quads), looked up once per device.
hipError_t euler_scratch(double** out);
// t2h_eltwise.hip
hipError_t launch_activation(const EltArgs& a, hipStream_t s);
hipError_t launch_gate_residual(const EltArgs& a, hipStream_t s);
hipError_t launch_modulate(const EltArgs& a, hipStream_t s);
hipError_t launch_binop_rows(const EltArgs& a, hipStream_t s);
hipError_t launch_timestep(const float* t, void* out, int64_t n, int32_t dim, int32_t dtype,
                           const float* freqs_host, hipStream_t s);
hipError_t launch_offsets(const int32_t* coords, int64_t rows, int32_t coord_cols, int32_t nbatch,
                          int64_t* offsets, int64_t* first_bad, hipStream_t s);
hipError_t launch_modulation_add(const float* mod, const float* modulation, float* m, int64_t n,
                                 int64_t width, hipStream_t s);

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace t2h
