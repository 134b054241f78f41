/*
 * t2h.h — C ABI of libt2h.so: MI355X (gfx950) kernels for the fused per-token
 * ops of TRELLIS.2's flow-matching DiT blocks (LayerNorm + adaLN modulate,
 * multi-head QK RMSNorm, 3D RoPE from voxel coordinates, GELU-tanh + bias,
 * gated residual, sinusoidal timestep embedding), over dense token rows and
 * SparseTensor feature rows.
 *
 * Callers: the reference's Mojo host code through
 * `external_call["t2h_...", Int32](...)` behind its TRELLIS2_GPU switch
 * (trellis2_mojo/gpu/context.mojo:168-182), and the Python `t2h` package
 * (ctypes) used by the tests and bench.py.
 *
 * Conventions (every entry point):
 *   - Returns int32 status: T2H_OK (0) or a negative T2H_E* code; the message
 *     is in t2h_last_error() (thread-local, valid until the next call on the
 *     same thread).
 *   - Pointers are DEVICE pointers unless the name ends in `_host`. The
 *     t2h_h_* functions take HOST pointers only.
 *   - `stream` is a hipStream_t (NULL = the default stream). Device entry
 *     points only enqueue work: no allocation, no synchronisation, no host
 *     reads of device data. They are stateless and reentrant, with one
 *     exception: t2h_flow_euler_step_noalloc keeps its rescale statistics in
 *     one scratch array per GPU, so its calls that overlap on one GPU (other
 *     streams or threads) mix each other's statistics and are not reentrant.
 *   - `dtype` (T2H_F32 / T2H_F16 / T2H_BF16) is the storage type of the token
 *     tensors; all arithmetic is f32. Parameter vectors (shift, scale, gate,
 *     bias, gamma, weight) are always f32, as in the reference.
 *   - Output may alias input (in place) wherever the entry point says so.
 *   - rows == 0 is a valid no-op (empty tensors).
 *
 * Batch map — which row of a [B, C] parameter array applies to token row r
 * (the reference's `batch_broadcast_map`, sparse/basic.mojo:149-155, and the
 * dense [N, L, C] broadcast of modules/nn.mojo:660-689):
 *   offsets != NULL      b(r) = the b with offsets[b] <= r < offsets[b+1]
 *                        (int64 device [nbatch+1], VarLenTensor offsets);
 *   else rows_per_batch  b(r) = r / rows_per_batch   (dense [N, L, C], L);
 *   else                 b(r) = 0.
 * Parameter row b starts at param + b * p_stride (p_stride 0 = cols), so the
 * six adaLN chunks can be read in place from one [B, 6C] modulation tensor.
 */
#ifndef T2H_H
#define T2H_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define T2H_VERSION 10000 /* 1.0.0 */

/* storage types */
#define T2H_F32 0
#define T2H_F16 1
#define T2H_BF16 2

/* status codes */
#define T2H_OK 0
#define T2H_EINVAL (-1)          /* bad argument (shape mismatch, NULL, range) */
#define T2H_EUNSUPPORTED (-2)    /* valid but unsupported shape/dtype */
#define T2H_EHIP (-3)            /* HIP runtime error */
#define T2H_EBATCH_ORDER (-4)    /* coords: batches not ordered/contiguous */
#define T2H_EBATCH_RANGE (-5)    /* coords: batch index out of range */
#define T2H_EDEVICE (-6)         /* device is not gfx950 */

/* LayerNorm epilogue modes (gpu/block.mojo:47-83 modes 1/2, plus plain) */
#define T2H_LN_PLAIN 0     /* y = LN(x) */
#define T2H_LN_MODULATE 1  /* y = LN(x) * (1 + p1[b]) + p0[b]   (p0 shift, p1 scale) */
#define T2H_LN_AFFINE 2    /* y = LN(x) * p0 + p1               (p0 weight, p1 bias) */

/* activation kinds: modules/nn.mojo:582-585 */
#define T2H_ACT_RELU 0
#define T2H_ACT_SILU 1
#define T2H_ACT_GELU 2
#define T2H_ACT_GELU_TANH 3
#define T2H_ACT_NONE (-1)        /* t2h_linear: no activation */

/* binary ops: sparse/tensor.mojo:4-7 */
#define T2H_OP_ADD 0
#define T2H_OP_SUB 1
#define T2H_OP_MUL 2
#define T2H_OP_DIV 3
#define T2H_OP_RSUB 4   /* other - x: _binop_scalar(reverse=True), sparse/tensor.mojo:200-203 */
#define T2H_OP_RDIV 5   /* other / x */

/* limits */
#define T2H_MAX_HALF_HEAD 128      /* head_dim <= 256 */
#define T2H_MAX_POS_DIM 4
#define T2H_MAX_TIMESTEP_HALF 512  /* frequency_embedding_size <= 1024 */

/* ---- library ---------------------------------------------------------- */
int32_t t2h_version(void);
const char* t2h_last_error(void);
/* Select `device` and check that it is a gfx950 (MI355X) GPU.
 * Replaces GpuContext construction + self-test (gpu/context.mojo:116-182). */
int32_t t2h_device_init(int32_t device);

/* ---- LayerNorm + adaLN modulate -----------------------------------------
 * Replaces: LayerNorm32.forward (modules/nn.mojo:314-369) fused with
 * modulate (modules/nn.mojo:660-689) / _mod_shift_scale
 * (sparse/transformer/modulated.mojo:60-65, batch-gathered), and the Metal
 * kernel ln_mod_rows (gpu/block.mojo:47-83).
 * x, out: [rows, cols] of dtype (out may alias x). Per row: mean, biased
 * variance (two-pass), inv = 1/sqrt(var + eps), n = (x - mean) * inv, then
 * the `mode` epilogue. For T2H_LN_AFFINE the batch map is ignored. */
int32_t t2h_ln_modulate(const void* x, void* out, int64_t rows, int32_t cols,
                        int32_t dtype, float eps, int32_t mode,
                        const float* p0, const float* p1, int64_t p_stride,
                        const int64_t* offsets, int32_t nbatch,
                        int64_t rows_per_batch, void* stream);

/* Modulate alone: out = fl(x * fl(1 + scale[b])) + shift[b], bit-exact with
 * modules/nn.mojo:680-684 and sparse/transformer/modulated.mojo:60-65. */
int32_t t2h_modulate(const void* x, void* out, int64_t rows, int32_t cols,
                     int32_t dtype, const float* shift, const float* scale,
                     int64_t p_stride, const int64_t* offsets, int32_t nbatch,
                     int64_t rows_per_batch, void* stream);

/* SparseTensor.elemwise_batch (sparse/basic.mojo:433-436 ->
 * Tensor._binop_rows sparse/tensor.mojo:205-219): out[r,:] = x[r,:] OP
 * other[b(r), :]; other_cols == cols or 1 (a per-batch scalar). With one
 * batch and other_cols 1 this is Tensor._binop_scalar (sparse/tensor.mojo:
 * 200-203); T2H_OP_RSUB / T2H_OP_RDIV are its reverse forms. Bit-exact. */
int32_t t2h_binop_rows(const void* x, const float* other, void* out,
                       int64_t rows, int32_t cols, int32_t other_cols,
                       int32_t dtype, int32_t op, const int64_t* offsets,
                       int32_t nbatch, int64_t rows_per_batch, void* stream);

/* ---- multi-head QK RMSNorm + 3D RoPE ------------------------------------
 * Replaces: MultiHeadRMSNorm.forward (sparse/attention/modules.mojo:49-102),
 * apply_rotary_embedding (modules/rope.mojo:64-88),
 * SparseRotaryPositionEmbedder.embed (sparse/attention/rope.mojo:128-134) and
 * the Metal kernels bias_rms_rope_qkv / bias_rms_q
 * (gpu/attention.mojo:507-563, 596-631), in the order bias -> RMS -> RoPE
 * (modules/attention.mojo:122-130; sparse/attention/modules.mojo:206-212).
 *
 * q_in/k_in/q_out/k_out: [rows, heads, head_dim] with row strides in_stride /
 * out_stride (elements; 0 = heads*head_dim), so q and k can be views into a
 * packed qkv [rows, 3, H, D] buffer (stride 3*H*D). Either q or k may be NULL.
 * In place when q_out == q_in / k_out == k_in.
 * bias_q/bias_k: [H*D] f32 or NULL. gamma_q/gamma_k: [H, D] f32; both NULL =
 * no RMS norm. RMS: n = max(sqrt(sum x^2), 1e-12); y = x / n * gamma * scale,
 * scale = f32(sqrt(f64(head_dim))).
 * RoPE (use_rope != 0), interleaved pairs (x[2p], x[2p+1]) rotated by
 * (cos, sin) of slot p; slots p >= pos_dim * freq_dim are identity.
 * The angle of slot p = pos[p / freq_dim] * freqs_host[p % freq_dim] in f32,
 * where freqs_host is the caller's HOST table (RotaryPositionEmbedder.freqs,
 * modules/rope.mojo:33-37; freq_dim <= 128). Position source, first non-NULL:
 *   phases:  precomputed [phase_rows, D/2, 2] f32, row (r % phase_rows)
 *   coords:  int32 [rows, coord_cols]; pos[a] = coords[r, 1 + a]
 *            (sparse/attention/rope.mojo:61)
 *   grid_res: R > 0, dense 'ij' grid, l = r % R^3 -> (l/R^2, (l/R)%R, l%R)
 *            (models/sparse_structure_flow.mojo:139-149).
 */
int32_t t2h_qk_rmsnorm_rope(const void* q_in, const void* k_in, void* q_out,
                            void* k_out, int64_t rows, int64_t in_stride,
                            int64_t out_stride, int32_t heads, int32_t head_dim,
                            int32_t dtype, const float* bias_q,
                            const float* bias_k, const float* gamma_q,
                            const float* gamma_k, int32_t use_rope,
                            const float* freqs_host, int32_t freq_dim,
                            int32_t pos_dim, const float* phases,
                            int64_t phase_rows, const int32_t* coords,
                            int32_t coord_cols, int32_t grid_res, void* stream);

/* In place on a packed qkv GEMM output [rows, 3, H, D]: + bias (all three),
 * RMS q/k, RoPE q/k — exactly the Metal kernel bias_rms_rope_qkv
 * (gpu/attention.mojo:507-563; consts layout [3HD bias][HD gq][HD gk]).
 * bias may be NULL; gamma_q/gamma_k NULL = no RMS. */
int32_t t2h_qkv_bias_rmsnorm_rope(void* qkv, int64_t rows, int32_t heads,
                                  int32_t head_dim, int32_t dtype,
                                  const float* bias, const float* gamma_q,
                                  const float* gamma_k, int32_t use_rope,
                                  const float* freqs_host, int32_t freq_dim,
                                  int32_t pos_dim, const float* phases,
                                  int64_t phase_rows, const int32_t* coords,
                                  int32_t coord_cols, int32_t grid_res,
                                  void* stream);

/* ---- attention epilogue + head-major packing ------------------------------
 * Replaces the self-attention chain's bias_rms_rope_qkv followed by pack_q_z
 * and pack_kv_z (gpu/attention.mojo:507-563, 566-594, 634-662; sequence
 * 987-1013), and the cross chain's bias_rms_q + pack_q_z (596-631,
 * 1223-1234), in one pass that leaves q/k/v unmodified:
 *   q, k, v: [rows, H, D] rows in_stride elements apart (0 = H*D); views of a
 *            packed qkv [rows, 3, H, D] use in_stride 3*H*D. NULL = absent.
 *   q, k: + bias, RMS (gamma_q/gamma_k, both or none; n = max(|x|, 1e-12),
 *         x / n * gamma * sqrt(f32(D))), RoPE (positions as in
 *         t2h_qk_rmsnorm_rope); v: + bias only.
 *   qh    [H, mp, D] = q * (1 / sqrt(f32(D)))           (NULL = skip)
 *   k_out [H, D, lp] (k_transposed = 1, the reference's kt; lp % 8 == 0)
 *         or [H, lp, D] (k_transposed = 0)               (NULL = skip)
 *   vh    [H, lp, D]                                     (NULL = skip)
 * Rows rows..mp-1 of qh and rows..lp-1 of k_out / vh are written as zeros.
 * head_dim 64 or 128. Outputs must not overlap the inputs. */
int32_t t2h_attn_pack(const void* q, const void* k, const void* v,
                      int64_t in_stride, int64_t rows, int32_t heads,
                      int32_t head_dim, int32_t dtype, const float* bias_q,
                      const float* bias_k, const float* bias_v,
                      const float* gamma_q, const float* gamma_k,
                      int32_t use_rope, const float* freqs_host,
                      int32_t freq_dim, int32_t pos_dim, const float* phases,
                      int64_t phase_rows, const int32_t* coords,
                      int32_t coord_cols, int32_t grid_res, void* qh,
                      int64_t mp, void* k_out, void* vh, int64_t lp,
                      int32_t k_transposed, void* stream);

/* ---- linear fused with the gated residual join ------------------------------
 * out[t, n] = res[t, n] + fl(fl(sum_k x[t, k] * w[n, k] + bias[n]) * gate[b(t), n])
 * (gate NULL: res + fl(acc + bias)): the block's residual join in the store
 * of the GEMM that makes h.
 * Replaces: the out linear's GpuLinear.enqueue_gemm (attention out-projection,
 * the MLP's lin2: gpu/linear.mojo:535-560, 776-809) followed by
 * gate_add_bias_rows (gpu/block.mojo:86-110, sequence 317-397), and the CPU
 * form x + h.elemwise_batch(gate, MUL) with per-batch gate rows
 * (sparse/transformer/modulated.mojo:214-226).
 * x, w, bias, shapes and alignment as t2h_linear; res and out [rows,
 * out_features] (rows ldo elements apart) in out_dtype (f32 or dtype); out
 * may alias res. gate rows gate_stride apart (0 = out_features), batch of a
 * row from offsets [nbatch + 1] or rows_per_batch, as t2h_gate_residual. */
int32_t t2h_linear_gate_residual(const void* x, int64_t ldx, const void* w,
                                 const float* bias, const void* res,
                                 void* out, int64_t ldo, int64_t rows,
                                 int32_t in_features, int32_t out_features,
                                 int32_t dtype, int32_t out_dtype,
                                 const float* gate, int64_t gate_stride,
                                 const int64_t* offsets, int32_t nbatch,
                                 int64_t rows_per_batch, void* stream);

/* ---- qkv linear fused with the attention epilogue and head-major pack -----
 * The self-attention chain's qkv GEMM, bias_rms_rope_qkv, pack_q_z and
 * pack_kv_z in one kernel: the GEMM's [rows, 3, H, D] output stays in
 * registers and only the packed operands are written.
 * Replaces: GpuLinear.enqueue_gemm of the qkv linear followed by
 * bias_rms_rope_qkv + pack_q_z + pack_kv_z (gpu/attention.mojo:983-1013;
 * kernels 507-563, 566-594, 634-662; gpu/linear.mojo:535-560).
 * x [rows, in_features] (rows ldx elements apart) and w [3*heads*head_dim,
 * in_features] (the qkv linear's [out, in] weight), both f16 or both bf16,
 * f32 sums. Biases, gammas, RoPE sources and outputs as t2h_attn_pack; all
 * three outputs are required. head_dim 128 with heads even, or head_dim 64
 * with heads a multiple of 4 (a wave's 128 features are one head or two);
 * in_features % 64 == 0. */
int32_t t2h_qkv_linear_pack(const void* x, int64_t ldx, const void* w,
                            int64_t rows, int32_t in_features, int32_t heads,
                            int32_t head_dim, int32_t dtype,
                            const float* bias_q, const float* bias_k,
                            const float* bias_v, const float* gamma_q,
                            const float* gamma_k, int32_t use_rope,
                            const float* freqs_host, int32_t freq_dim,
                            int32_t pos_dim, const float* phases,
                            int64_t phase_rows, const int32_t* coords,
                            int32_t coord_cols, int32_t grid_res, void* qh,
                            int64_t mp, void* k_out, void* vh, int64_t lp,
                            int32_t k_transposed, void* stream);

/* Host function (no device work): the embedders' frequency table
 * freqs[j] = f32(freq_lo) / f32(freq_hi) ** (f32(j) / f32(freq_dim)),
 * freq_dim = head_dim / 2 / dim, in f32 with libm powf — the constructor of
 * RotaryPositionEmbedder / SparseRotaryPositionEmbedder (modules/rope.mojo:
 * 24-37, sparse/attention/rope.mojo:26-39). Writes min(freq_dim, capacity)
 * entries and returns freq_dim, or a negative status (odd head_dim). */
int32_t t2h_rope_freqs(int32_t head_dim, int32_t dim, double freq_lo,
                       double freq_hi, float* freqs_host, int32_t capacity);

/* Phase table [rows, head_dim/2, 2] f32 (cos, sin): replaces
 * RotaryPositionEmbedder.forward (modules/rope.mojo:39-61; positions f32
 * [rows, pos_dim]) and SparseRotaryPositionEmbedder._compute_phases
 * (sparse/attention/rope.mojo:48-66; int32 coords). Source: positions, else
 * coords, else grid_res. */
int32_t t2h_rope_phases(float* phases_out, int64_t rows, int32_t head_dim,
                        const float* freqs_host, int32_t freq_dim,
                        int32_t pos_dim, const float* positions,
                        const int32_t* coords, int32_t coord_cols,
                        int32_t grid_res, void* stream);

/* ---- activation (+ bias) -------------------------------------------------
 * Replaces: activation(x, kind) (modules/nn.mojo:588-647) applied to a
 * linear's output with its bias (nn.mojo:123-133), i.e. act(x + bias[col]),
 * and the Metal kernel gelu_tanh_bias (gpu/linear.mojo:662-684).
 * x, out: [rows, cols] (out may alias x); bias [cols] f32 or NULL. */
int32_t t2h_activation(const void* x, void* out, const float* bias,
                       int64_t rows, int32_t cols, int32_t dtype, int32_t kind,
                       void* stream);

/* ---- weight GEMM on the matrix cores ---------------------------------------
 * out[t, n] = act(sum_k x[t, k] * w[n, k] + bias[n]): a linear layer with
 * the bias and activation applied in the GEMM's store.
 * Replaces: GpuLinear.enqueue_gemm (gpu/linear.mojo:535-560; c[m, co] =
 * a[m, ci] @ W^T) and, with act = T2H_ACT_GELU_TANH, the MLP's first linear
 * followed by gelu_tanh_bias (gpu/linear.mojo:662-684, 776-809).
 * x [rows, in_features] (rows ldx elements apart), w [out_features,
 * in_features] contiguous (the checkpoint's [out, in] layout), both f16 or
 * both bf16 (dtype); f32 products and sums, as the reference's 16-bit-weight
 * kernel gemm_tiled_f16sh (gpu/linear.mojo:326-388). bias [out_features] f32
 * or NULL; act T2H_ACT_* or T2H_ACT_NONE. out [rows, out_features] (rows ldo
 * elements apart) in out_dtype = T2H_F32 or dtype.
 * Shapes: out_features % 256 == 0, in_features % 64 == 0, ldx % 8 == 0,
 * ldo % 8 (16-bit out) or % 4 (f32 out) == 0; x, w, bias, out 16-byte
 * aligned. */
int32_t t2h_linear(const void* x, int64_t ldx, const void* w,
                   const float* bias, void* out, int64_t ldo, int64_t rows,
                   int32_t in_features, int32_t out_features, int32_t dtype,
                   int32_t out_dtype, int32_t act, void* stream);

/* ---- gated residual ------------------------------------------------------
 * Replaces: `y + _gate(h, g)` (modules/transformer/modulated.mojo:22-33,
 * 60-69, 192-200), `x + h.elemwise_batch(gate, MUL)`
 * (sparse/transformer/modulated.mojo:214-226) and the Metal kernel
 * gate_add_bias_rows (gpu/block.mojo:86-110):
 *   out = x + fl(fl(h + bias) * gate[b(r)])       (each step one rounding)
 * bias NULL: no bias step; gate NULL: ungated (x + h); x NULL: out = the gated
 * term alone (`_gate`). out may alias x or h. Bit-exact with the reference. */
int32_t t2h_gate_residual(const void* x, const void* h, void* out,
                          const float* bias, const float* gate,
                          int64_t p_stride, int64_t rows, int32_t cols,
                          int32_t dtype, const int64_t* offsets,
                          int32_t nbatch, int64_t rows_per_batch, void* stream);

/* Fused block join: x_out = x + fl(fl(h + bias) * gate[b]) (as above, stored
 * in dtype), then y_out = LN(x_out) with the `mode` epilogue (as
 * t2h_ln_modulate, p0/p1). One HBM pass instead of two. x_out may alias x. */
int32_t t2h_gate_residual_ln_modulate(
    const void* x, const void* h, void* x_out, void* y_out, const float* bias,
    const float* gate, int64_t gate_stride, float eps, int32_t mode,
    const float* p0, const float* p1, int64_t p_stride, int64_t rows,
    int32_t cols, int32_t dtype, const int64_t* offsets, int32_t nbatch,
    int64_t rows_per_batch, void* stream);

/* ---- flow-matching Euler sampler step ------------------------------------
 * Replaces the per-step tensor math of FlowEulerSampler._sample_impl
 * (samplers/flow_euler.mojo:196-210) with _inference's CFG combine and CFG
 * rescale (151-181, _rescale_pred 75-149) over one flat state of rows x
 * row_size elements (x_t, v_pos, v_neg, x_prev, pred_x0 all of dtype):
 *   pred = v_pos                                     (v_neg NULL, or g == 1)
 *        = v_neg                                     (g == 0)
 *        = fl(v_pos * f32(g)) + fl(v_neg * f32(1-g))  (otherwise)
 *   with guidance_rescale > 0 and both predictions, pred is rescaled so that
 *   each segment's x_0 has the positive branch's std (segments: one per row,
 *   unbiased std; or the host token offsets seg_offsets_host [n] in rows,
 *   biased std; rows outside them get pred 0, as in the reference);
 *   x_prev  = fl(x_t - fl(pred * f32(t - t_prev)))
 *   pred_x0 = fl(x_t * f32(1 - sigma_min)) - fl(pred * f32(sigma_min + (1 - sigma_min) t))
 *            (NULL = not written)
 * The elementwise results are bit-exact with the reference; the rescale's
 * std is summed in f64 (the reference sums serially in f32), in a fixed
 * order, so repeated calls give the same bits. The rescale needs a device
 * workspace of t2h_flow_euler_workspace() bytes (16-byte aligned, any
 * contents); calls that share a workspace must not overlap. With one
 * segment (rows == 1 dense, or two seg offsets) on whole 16-byte vectors
 * and a workspace of that size, a state that fits the registers of the
 * resident grid (up to ~7M f32 elements on MI355X) is rescaled in one
 * launch whose blocks meet at a grid barrier in the workspace; its result
 * does not depend on other streams' work (a block that cannot be resident
 * in time leaves its share to the grid's reducing block, which only costs
 * time). A smaller workspace (at least the statistics partials', as the
 * error names) gives the two-launch form. */
int64_t t2h_flow_euler_workspace(int64_t rows, int64_t row_size,
                                 int32_t n_seg_offsets);
int32_t t2h_flow_euler_step(const void* x_t, const void* v_pos,
                            const void* v_neg, void* x_prev, void* pred_x0,
                            int64_t rows, int64_t row_size, int32_t dtype,
                            double t, double t_prev, double sigma_min,
                            double guidance_strength, double guidance_rescale,
                            const int64_t* seg_offsets_host,
                            int32_t n_seg_offsets, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* No counterpart in the reference: t2h_flow_euler_step for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments without the
 * workspace: the rescale's statistics (and the one-launch form's barrier)
 * go to a scratch array built into the library, 512 KB per GPU (16,384
 * statistics blocks: every varlen split of up to 64 segments, or up to
 * 16,384 dense rows of <= 16,384 elements each; larger dense states return
 * T2H_EUNSUPPORTED). It allocates nothing, and
 * its results equal t2h_flow_euler_step's bit for bit. Every call on a GPU
 * shares that GPU's scratch, so calls that overlap on one GPU (other
 * streams, other threads) race; stream-ordered calls do not. Call
 * t2h_device_init first to do the one-time per-device scratch lookup
 * outside any capture. */
int32_t t2h_flow_euler_step_noalloc(const void* x_t, const void* v_pos,
                                    const void* v_neg, void* x_prev,
                                    void* pred_x0, int64_t rows,
                                    int64_t row_size, int32_t dtype, double t,
                                    double t_prev, double sigma_min,
                                    double guidance_strength,
                                    double guidance_rescale,
                                    const int64_t* seg_offsets_host,
                                    int32_t n_seg_offsets, void* stream);

/* ---- resident-block glue over one const buffer ---------------------------
 * The device-resident DiT cross block keeps its per-block glue constants in
 * one f32 buffer `consts` of 12*C floats (gpu/block.mojo:255-289): pairs of
 * [C] vectors at offsets 0, 2C, 4C, 6C, 8C, 10C =
 *   (shift1, scale1) (self_out bias, gate1) (norm2 weight, bias)
 *   (cross_out bias, 0) (shift3, scale3) (mlp2 bias, gate3).
 * `off` selects a pair: consts[off : off+C] and consts[off+C : off+2C].
 * All three calls take the reference kernels' arguments in their order, plus
 * the storage dtype and the stream. eps is the blocks' 1e-6 (block.mojo:44). */

/* Replaces: Metal ln_mod_rows (gpu/block.mojo:47-83). mode 1: dst =
 * LN(x)*(1+consts[off+C+i]) + consts[off+i]; mode 2 (affine): dst =
 * LN(x)*consts[off+i] + consts[off+C+i]. dst may alias x. */
int32_t t2h_ln_mod_rows(const void* x, void* dst, const float* consts,
                        int64_t rows, int32_t c, int32_t off, int32_t mode,
                        int32_t dtype, void* stream);

/* Replaces: Metal gate_add_bias_rows (gpu/block.mojo:86-110), in place:
 * x += fl(h + consts[off+i]) * consts[off+C+i]   (use_gate 1)
 * x += fl(h + consts[off+i])                     (use_gate 0). Bit-exact. */
int32_t t2h_gate_add_bias_rows(void* x, const void* h, const float* consts,
                               int64_t rows, int32_t c, int32_t off,
                               int32_t use_gate, int32_t dtype, void* stream);

/* Replaces the block's join + next norm pair, gate_add_bias_rows(join_off,
 * use_gate) followed by ln_mod_rows(norm_off, mode) (gpu/block.mojo:324-349
 * and 356-381), in one HBM pass: x updated in place, dst = the normed rows.
 * dst must not alias x or h. */
int32_t t2h_block_join_ln(void* x, const void* h, void* dst,
                          const float* consts, int64_t rows, int32_t c,
                          int32_t join_off, int32_t use_gate, int32_t norm_off,
                          int32_t mode, int32_t dtype, void* stream);

/* ---- timestep embedding --------------------------------------------------
 * Replaces TimestepEmbedder.timestep_embedding
 * (models/sparse_structure_flow.mojo:60-76): t [n] f32 -> out [n, dim]:
 * half = dim/2, freq_j = exp(-f32(log(max_period)) * j / half) (f32),
 * out[:, j] = cos(t * freq_j), out[:, half + j] = sin(t * freq_j); odd dim
 * leaves a zero last column. dim/2 <= T2H_MAX_TIMESTEP_HALF. */
int32_t t2h_timestep_embedding(const float* t, void* out, int64_t n,
                               int32_t dim, int32_t dtype, double max_period,
                               void* stream);

/* ---- SparseTensor layout ---------------------------------------------------
 * Replaces SparseTensor._cal_offsets (sparse/basic.mojo:321-339): offsets
 * [nbatch+1] int64 from coords[:, 0] (int32 [rows, coord_cols]).
 * first_bad (int64 device scalar) receives INT64_MAX when valid, else
 * (r << 1) | kind for the first offending row r (kind 0: batch below the
 * previous row's — not ordered/contiguous; kind 1: batch < 0 or >= nbatch),
 * the reference's two `raise` branches in its row order. Offsets are
 * meaningful only when first_bad == INT64_MAX. */
int32_t t2h_coords_to_offsets(const int32_t* coords, int64_t rows,
                              int32_t coord_cols, int32_t nbatch,
                              int64_t* offsets, int64_t* first_bad,
                              void* stream);

/* Modulation.chunks, share_mod branch (sparse/transformer/modulated.mojo:
 * 41-48): m[r, j] = mod[r, j] + modulation[j] over [n, width] (f32). */
int32_t t2h_modulation_add(const float* mod, const float* modulation, float* m,
                           int64_t n, int64_t width, void* stream);

/* ---- host-pointer convenience (synchronous) ------------------------------
 * For the unchanged Tensor[F32] API (host memory in, fresh host tensor out,
 * modules/nn.mojo:314-320): copy in, run the device entry point on the
 * default stream, copy out. These allocate device memory per call; the
 * device-pointer entry points above are the hot path. All f32. */
int32_t t2h_h_ln_modulate(const float* x_host, float* out_host, int64_t rows,
                          int32_t cols, float eps, int32_t mode,
                          const float* p0_host, const float* p1_host,
                          const int64_t* offsets_host, int32_t nbatch,
                          int64_t rows_per_batch);
int32_t t2h_h_qk_rmsnorm_rope(const float* q_host, const float* k_host,
                              float* q_out_host, float* k_out_host,
                              int64_t rows, int32_t heads, int32_t head_dim,
                              const float* gamma_q_host,
                              const float* gamma_k_host, int32_t use_rope,
                              const float* freqs_host, int32_t freq_dim,
                              int32_t pos_dim, const float* phases_host,
                              int64_t phase_rows, const int32_t* coords_host,
                              int32_t coord_cols, int32_t grid_res);
int32_t t2h_h_activation(const float* x_host, float* out_host,
                         const float* bias_host, int64_t rows, int32_t cols,
                         int32_t kind);
int32_t t2h_h_gate_residual(const float* x_host, const float* h_host,
                            float* out_host, const float* bias_host,
                            const float* gate_host, int64_t rows, int32_t cols,
                            const int64_t* offsets_host, int32_t nbatch,
                            int64_t rows_per_batch);
int32_t t2h_h_timestep_embedding(const float* t_host, float* out_host,
                                 int64_t n, int32_t dim, double max_period);
int32_t t2h_h_coords_to_offsets(const int32_t* coords_host, int64_t rows,
                                int32_t coord_cols, int32_t nbatch,
                                int64_t* offsets_host);

#ifdef __cplusplus
}
#endif
#endif /* T2H_H */
