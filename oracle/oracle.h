/*
 * CPU oracle for the fused per-token DiT ops: a plain-C restatement of the
 * reference's Mojo CPU path (mrvoll98/trellis2-mojo, read as text only).
 *
 * TEST INFRASTRUCTURE ONLY. The product (libt2h.so and the t2h package)
 * never links, loads or calls this code; only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg use it, as the checker.
 *
 * Every function names the reference file:line it follows. Arithmetic is f32
 * with the reference's operation order and rounding steps (the library is
 * built with -ffp-contract=off so a*b+c is two roundings, as in Mojo without
 * fast-math). Transcendentals come from the host libm (glibc); the reference
 * uses Mojo's std.math, which no file under the reference pins, so those
 * values agree to a few ulp, not bit for bit.
 *
 * Threading mirrors the reference: functions the reference runs serially run
 * serially; the three it runs under `parallelize` (activation, MultiHeadRMSNorm,
 * sparse RoPE rotate) take an `nthreads` argument and use OpenMP over the same
 * chunks (32768 elements / 64 rows) above the same 2^17-element threshold.
 * Parallel chunks write disjoint outputs, so results do not depend on nthreads.
 */
#ifndef T2H_ORACLE_H
#define T2H_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded inputs: trellis2_mojo/rng.mojo:17-52 ---------------------- */
typedef struct { uint64_t state; } orc_rng;
void orc_rng_init(orc_rng* r, uint64_t seed);            /* rng.mojo:22-28 */
uint64_t orc_rng_next_u64(orc_rng* r);                    /* rng.mojo:30-36 */
double orc_rng_next_f64(orc_rng* r);                      /* rng.mojo:38-39 */
double orc_rng_normal(orc_rng* r);                        /* rng.mojo:41-46 */
/* randn (rng.mojo:49-52) scaled: out[i] = (float)(mean + std * normal()).
 * With mean 0, std 1 this is exactly the reference's randn. */
void orc_randn(orc_rng* r, float* out, int64_t n, double mean, double std);
void orc_uniform(orc_rng* r, float* out, int64_t n, double lo, double hi);

/* ---- LayerNorm32.forward: modules/nn.mojo:314-369 ----------------------- */
int orc_layernorm(const float* x, float* out, int64_t rows, int64_t c,
                  double eps, int affine, const float* w, const float* b);

/* ---- modulate: modules/nn.mojo:660-689 (x [N,L,C], shift/scale [N,C]) --- */
int orc_modulate(const float* x, const float* shift, const float* scale,
                 float* out, int64_t n, int64_t l, int64_t c);

/* ---- SparseTensor layout: sparse/basic.mojo:321-339 (_cal_offsets) ------
 * Returns 0, or -1 when batches are not ordered/contiguous, -2 when a batch
 * index is out of range (the two `raise Error` branches). */
int orc_cal_offsets(const int32_t* coords, int64_t rows, int64_t ncols,
                    int64_t batch_size, int64_t* offsets /* [B+1] */);
/* VarLenTensor.batch_broadcast_map: sparse/basic.mojo:149-155 */
void orc_batch_broadcast_map(const int64_t* offsets, int64_t batch_size,
                             int64_t* row_map);

/* ---- Tensor._binop_rows: sparse/tensor.mojo:205-219 (+ _op_span ops) ----
 * out[r,:] = x[r,:] OP other[row_map[r], :] ; other row size = c or 1.
 * op: 0 add, 1 sub, 2 mul, 3 div (sparse/tensor.mojo:4-7). */
int orc_binop_rows(const float* x, const float* other, const int64_t* row_map,
                   float* out, int64_t rows, int64_t c, int64_t other_c, int op);
/* Tensor._binop_scalar(v, op, reverse): x OP v elementwise, v OP x when reverse */
void orc_binop_scalar(const float* x, float v, float* out, int64_t n, int op, int reverse);
/* Tensor._binop_flat: x OP y elementwise (sparse/tensor.mojo:193-198) */
void orc_binop_flat(const float* x, const float* y, float* out, int64_t n, int op);

/* _mod_shift_scale: sparse/transformer/modulated.mojo:60-65 */
int orc_mod_shift_scale(const float* h, const float* shift, const float* scale,
                        const int64_t* offsets, int64_t batch_size,
                        float* out, int64_t rows, int64_t c);

/* Modulation.chunks, share_mod branch: sparse/transformer/modulated.mojo:41-48
 * m[r, j] = mod[r, j] + modulation[j] over [n, width]. */
void orc_modulation_add(const float* mod, const float* modulation, float* m,
                        int64_t n, int64_t width);

/* ---- MultiHeadRMSNorm.forward: sparse/attention/modules.mojo:49-102 ------ */
int orc_multihead_rmsnorm(const float* x, const float* gamma, float* out,
                          int64_t rows, int64_t h, int64_t d, int nthreads);
/* scale = Float32(Float64(dim) ** 0.5): sparse/attention/modules.mojo:47 */
float orc_rmsnorm_scale(int64_t d);

/* ---- RoPE: modules/rope.mojo:17-88, sparse/attention/rope.mojo:20-134 --- */
/* freqs[j] = f32(lo) / f32(hi) ** (f32(j)/f32(freq_dim)) (rope.mojo:35-37).
 * Returns freq_dim = head_dim / 2 / dim. */
int64_t orc_rope_freqs(int64_t head_dim, int64_t dim, double freq_lo,
                       double freq_hi, float* freqs);
/* RotaryPositionEmbedder.forward (rope.mojo:39-61): positions f32 [L, dim]
 * -> phases [L, head_dim/2, 2] (cos, sin), pad slots (1, 0). */
int orc_rope_phases_from_positions(const float* pos, int64_t l, int64_t dim,
                                   int64_t head_dim, const float* freqs,
                                   int64_t freq_dim, float* phases);
/* SparseRotaryPositionEmbedder._compute_phases (sparse rope.mojo:48-66):
 * coords int32 [N, ncols] (col 0 = batch, cols 1..dim = position). */
int orc_rope_phases_from_coords(const int32_t* coords, int64_t n, int64_t ncols,
                                int64_t dim, int64_t head_dim, const float* freqs,
                                int64_t freq_dim, float* phases);
/* meshgrid(indexing='ij') over R^3, l = i*R^2 + j*R + k:
 * models/sparse_structure_flow.mojo:139-149 */
void orc_grid_positions(int64_t r, float* pos /* [R^3, 3] */);
/* apply_rotary_embedding (rope.mojo:64-88): x [N, L, H, D], phases [L, D/2, 2] */
int orc_apply_rotary(const float* x, const float* phases, float* out,
                     int64_t n, int64_t l, int64_t h, int64_t d);
/* SparseRotaryPositionEmbedder._rotate (sparse rope.mojo:76-126):
 * feats [N, H, D], phases [N, D/2, 2]. */
int orc_rope_rotate(const float* feats, const float* phases, float* out,
                    int64_t n, int64_t h, int64_t d, int nthreads);

/* ---- activation: modules/nn.mojo:588-647 (kinds nn.mojo:582-585) ------- */
int orc_activation(const float* x, float* out, int64_t n, int kind, int nthreads);
/* linear's bias add (nn.mojo:123-133, 157-158): v = acc + b[col] */
void orc_add_bias(const float* x, const float* bias, float* out,
                  int64_t rows, int64_t c);

/* ---- _gate: modules/transformer/modulated.mojo:22-33 ------------------- */
void orc_gate(const float* x, const float* g, float* out,
              int64_t n, int64_t l, int64_t c);

/* ---- weight GEMM: gpu/linear.mojo:108-160 (gemm_tiled), 326-388 -------
 * (gemm_tiled_f16sh). c[m, n] = sum_k a[m, k] * w[n, k], w in the
 * checkpoint layout [n, k] (GpuLinear uploads W^T, linear.mojo:466-500; the
 * sum is the same). Each output accumulates its k in increasing order with
 * one f32 rounding per product and per add, as one thread of the reference
 * kernel does (its kb/kk loops walk k in order). With 16-bit-valued inputs
 * (the f16sh kernel rounds both operands to f16) every product is exact.
 * Rows are independent: OpenMP over rows with nthreads (results do not
 * depend on nthreads). */
void orc_linear(const float* a, const float* w, float* c, int64_t m,
                int64_t n, int64_t k, int nthreads);

/* ---- head-major attention packs: gpu/attention.mojo:566-594, 634-662 -- */
/* qh [h, mp, d] = q rows (`stride` apart, head z at z*d) * 1/sqrt(f32(d));
 * rows l..mp-1 zero. */
void orc_pack_q(const float* qkv, float* qh, int64_t l, int64_t h, int64_t d,
                int64_t mp, int64_t stride);
/* qkv [l, 3, h, d] parts 1/2 -> kt [h, d, lp] (transposed) and vh [h, lp, d];
 * pad columns / rows l..lp-1 zero. */
void orc_pack_kv(const float* qkv, float* kt, float* vh, int64_t l, int64_t h,
                 int64_t d, int64_t lp);

/* ---- FlowEulerSampler elementwise math: samplers/flow_euler.mojo:56-149, 151-181, 196-210 */
/* x0 = fl(x * f32(1 - sigma_min)) - fl(v * f32(sigma_min + (1 - sigma_min) * t)) */
void orc_flow_v_to_xstart(const float* x, const float* v, float* out, int64_t n, double t, double sigma_min);
/* pred = fl(pos * f32(g)) + fl(neg * f32(1 - g)) */
void orc_flow_cfg(const float* pos, const float* neg, float* out, int64_t n, double g);
/* CFG rescale (_rescale_pred): segments [bounds[b], bounds[b+1]) of the flat
 * state, bounds = seg_offsets * row_size (varlen, biased std) when
 * nseg_offsets > 0, else one segment per row of row_size (unbiased std). */
void orc_flow_rescale(const float* x_t, const float* pred, const float* pred_pos, float* out, int64_t rows,
                      int64_t row_size, double t, double sigma_min, double guidance_rescale,
                      const int64_t* seg_offsets, int64_t nseg_offsets);
/* x_prev = fl(x - fl(v * f32(t - t_prev))) */
void orc_flow_step(const float* x, const float* v, float* out, int64_t n, double t, double t_prev);

/* ---- TimestepEmbedder.timestep_embedding: sparse_structure_flow.mojo:60-76 */
void orc_timestep_embedding(const float* t, int64_t n, int64_t dim,
                            double max_period, float* out /* [n, dim] */);

/* ---- f16 helpers for the f16-storage configs (RNE, IEEE binary16) ----- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_round_f16(const float* x, float* out, int64_t n); /* f32->f16->f32 */
void orc_round_bf16(const float* x, float* out, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
