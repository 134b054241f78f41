/*
 * CPU oracle (test infrastructure only) — plain-C restatement of the
 * reference's Mojo CPU path for the fused per-token DiT ops. See oracle.h for
 * the contract; each function cites the reference file:line it restates.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Mojo SIMD[F32, 8].reduce_add(): halves tree (lanes i and i+4, then i and
 * i+2, then 0 and 1). The bit-level order of Mojo's reduction is not pinned
 * by any reference test; this is the order LLVM's vector-reduce expansion
 * produces, and parity with it is tolerance-based. */
static float reduce_add8(const float v[8]) {
    float s4[4], s2[2];
    for (int i = 0; i < 4; ++i) s4[i] = v[i] + v[i + 4];
    for (int i = 0; i < 2; ++i) s2[i] = s4[i] + s4[i + 2];
    return s2[0] + s2[1];
}

/* ------------------------------------------------------------------------ */
/* rng.mojo:17-52                                                           */
/* ------------------------------------------------------------------------ */
void orc_rng_init(orc_rng* r, uint64_t seed) {
    /* rng.mojo:22-28: splitmix64 finaliser of seed + golden gamma */
    uint64_t z = seed + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    r->state = z ^ (z >> 31);
    if (r->state == 0) r->state = 0x9E3779B97F4A7C15ull;
}

uint64_t orc_rng_next_u64(orc_rng* r) {
    /* rng.mojo:30-36: xorshift64* */
    uint64_t x = r->state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    r->state = x;
    return x * 0x2545F4914F6CDD1Dull;
}

double orc_rng_next_f64(orc_rng* r) {
    /* rng.mojo:38-39: top 53 bits / 2^53 */
    return (double)(orc_rng_next_u64(r) >> 11) * (1.0 / 9007199254740992.0);
}

double orc_rng_normal(orc_rng* r) {
    /* rng.mojo:41-46: Box-Muller, cosine branch, u1 redrawn while 0 */
    double u1 = orc_rng_next_f64(r);
    while (u1 == 0.0) u1 = orc_rng_next_f64(r);
    double u2 = orc_rng_next_f64(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void orc_randn(orc_rng* r, float* out, int64_t n, double mean, double std) {
    /* rng.mojo:49-52 (Float32(rng.normal())); mean/std applied in f64 first */
    for (int64_t i = 0; i < n; ++i) {
        double v = orc_rng_normal(r);
        out[i] = (mean == 0.0 && std == 1.0) ? (float)v : (float)(mean + std * v);
    }
}

void orc_uniform(orc_rng* r, float* out, int64_t n, double lo, double hi) {
    for (int64_t i = 0; i < n; ++i) out[i] = (float)(lo + (hi - lo) * orc_rng_next_f64(r));
}

/* ------------------------------------------------------------------------ */
/* LayerNorm32.forward: modules/nn.mojo:314-369                             */
/* ------------------------------------------------------------------------ */
int orc_layernorm(const float* x, float* out, int64_t rows, int64_t c,
                  double eps, int affine, const float* w, const float* b) {
    if (c <= 0) return -1;
    const float epsf = (float)eps; /* Float32(self.eps), nn.mojo:349 */
    for (int64_t r = 0; r < rows; ++r) { /* serial over rows, nn.mojo:325 */
        const float* xr = x + r * c;
        float* orow = out + r * c;
        /* mean: 8-lane partial sums, reduce_add, scalar tail (nn.mojo:327-336) */
        float sv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int64_t i = 0;
        for (; i + 8 <= c; i += 8)
            for (int k = 0; k < 8; ++k) sv[k] += xr[i + k];
        float mean = reduce_add8(sv);
        for (; i < c; ++i) mean += xr[i];
        mean /= (float)c;
        /* biased variance, second pass (nn.mojo:337-348) */
        float vv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        i = 0;
        for (; i + 8 <= c; i += 8)
            for (int k = 0; k < 8; ++k) {
                float d = xr[i + k] - mean;
                vv[k] += d * d;
            }
        float variance = reduce_add8(vv);
        for (; i < c; ++i) {
            float d = xr[i] - mean;
            variance += d * d;
        }
        variance /= (float)c;
        float inv_std = 1.0f / sqrtf(variance + epsf); /* nn.mojo:349 */
        if (affine) { /* nn.mojo:351-360: (x-mean)*inv*w + b */
            for (i = 0; i < c; ++i) orow[i] = (xr[i] - mean) * inv_std * w[i] + b[i];
        } else {      /* nn.mojo:361-367 */
            for (i = 0; i < c; ++i) orow[i] = (xr[i] - mean) * inv_std;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* modulate: modules/nn.mojo:660-689                                        */
/* ------------------------------------------------------------------------ */
int orc_modulate(const float* x, const float* shift, const float* scale,
                 float* out, int64_t n, int64_t l, int64_t c) {
    for (int64_t b = 0; b < n; ++b) {
        const int64_t mb = b * c;
        for (int64_t j = 0; j < l; ++j) {
            const int64_t xb = (b * l + j) * c;
            for (int64_t ci = 0; ci < c; ++ci) /* x*(1+scale)+shift, nn.mojo:680-684 */
                out[xb + ci] = x[xb + ci] * (1.0f + scale[mb + ci]) + shift[mb + ci];
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* SparseTensor._cal_offsets: sparse/basic.mojo:321-339                     */
/* ------------------------------------------------------------------------ */
int orc_cal_offsets(const int32_t* coords, int64_t rows, int64_t ncols,
                    int64_t batch_size, int64_t* offsets) {
    for (int64_t b = 0; b <= batch_size; ++b) offsets[b] = 0;
    int64_t prev = -1;
    for (int64_t r = 0; r < rows; ++r) {
        int64_t b = coords[r * ncols];
        if (b < prev) return -1;                  /* basic.mojo:329-330 */
        if (b >= batch_size || b < 0) return -2;  /* basic.mojo:331-332 */
        prev = b;
        offsets[b + 1] += 1;                      /* counts[b] += 1 */
    }
    for (int64_t b = 0; b < batch_size; ++b) offsets[b + 1] += offsets[b]; /* cumsum */
    return 0;
}

void orc_batch_broadcast_map(const int64_t* offsets, int64_t batch_size, int64_t* row_map) {
    /* basic.mojo:149-155 */
    int64_t k = 0;
    for (int64_t b = 0; b < batch_size; ++b)
        for (int64_t i = offsets[b]; i < offsets[b + 1]; ++i) row_map[k++] = b;
}

/* _op_span / _opscalar_span element op (sparse/tensor.mojo:426-524) */
static inline float apply_op(float a, float b, int op) {
    switch (op) {
        case 0: return a + b;
        case 1: return a - b;
        case 2: return a * b;
        default: return a / b;
    }
}

int orc_binop_rows(const float* x, const float* other, const int64_t* row_map,
                   float* out, int64_t rows, int64_t c, int64_t other_c, int op) {
    /* sparse/tensor.mojo:205-219 */
    if (other_c != c && other_c != 1) return -1;
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t src = row_map[r];
        for (int64_t i = 0; i < c; ++i) {
            const float bv = (other_c == c) ? other[src * c + i] : other[src];
            out[r * c + i] = apply_op(x[r * c + i], bv, op);
        }
    }
    return 0;
}

void orc_binop_scalar(const float* x, float v, float* out, int64_t n, int op, int reverse) {
    /* _opscalar_span (sparse/tensor.mojo:469-524): x OP v, or v OP x when
     * reverse (only SUB and DIV have a reverse form; ADD and MUL ignore it) */
    for (int64_t i = 0; i < n; ++i)
        out[i] = (reverse && (op == 1 || op == 3)) ? apply_op(v, x[i], op) : apply_op(x[i], v, op);
}

void orc_binop_flat(const float* x, const float* y, float* out, int64_t n, int op) {
    for (int64_t i = 0; i < n; ++i) out[i] = apply_op(x[i], y[i], op);
}

int orc_mod_shift_scale(const float* h, const float* shift, const float* scale,
                        const int64_t* offsets, int64_t batch_size,
                        float* out, int64_t rows, int64_t c) {
    /* sparse/transformer/modulated.mojo:60-65:
     *   scaled = h.elemwise_batch(scale + 1, MUL); scaled.elemwise_batch(shift, ADD) */
    for (int64_t b = 0; b < batch_size; ++b) {
        for (int64_t r = offsets[b]; r < offsets[b + 1]; ++r) {
            for (int64_t i = 0; i < c; ++i) {
                const float sc1 = scale[b * c + i] + 1.0f;   /* _binop_scalar(1.0, ADD) */
                const float t = h[r * c + i] * sc1;          /* OP_MUL */
                out[r * c + i] = t + shift[b * c + i];       /* OP_ADD */
            }
        }
    }
    (void)rows;
    return 0;
}

void orc_modulation_add(const float* mod, const float* modulation, float* m,
                        int64_t n, int64_t width) {
    for (int64_t r = 0; r < n; ++r)
        for (int64_t j = 0; j < width; ++j) m[r * width + j] = mod[r * width + j] + modulation[j];
}

/* ------------------------------------------------------------------------ */
/* MultiHeadRMSNorm: sparse/attention/modules.mojo:37-102                   */
/* ------------------------------------------------------------------------ */
float orc_rmsnorm_scale(int64_t d) { return (float)pow((double)d, 0.5); }

static void rms_rows(const float* x, const float* gamma, float* out,
                     int64_t r0, int64_t r1, int64_t h, int64_t d, float sc) {
    for (int64_t r = r0; r < r1; ++r) {
        for (int64_t head = 0; head < h; ++head) {
            const int64_t base = (r * h + head) * d;
            const int64_t gbase = head * d;
            float accv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int64_t i = 0;
            for (; i + 8 <= d; i += 8)
                for (int k = 0; k < 8; ++k) accv[k] += x[base + i + k] * x[base + i + k];
            float norm = reduce_add8(accv);
            for (; i < d; ++i) norm += x[base + i] * x[base + i];
            norm = sqrtf(norm);
            if (norm < 1e-12f) norm = 1e-12f;  /* modules.mojo:84-85 */
            for (i = 0; i < d; ++i)            /* x / n * gamma * scale, left to right */
                out[base + i] = x[base + i] / norm * gamma[gbase + i] * sc;
        }
    }
}

int orc_multihead_rmsnorm(const float* x, const float* gamma, float* out,
                          int64_t rows, int64_t h, int64_t d, int nthreads) {
    const float sc = orc_rmsnorm_scale(d);
    const int64_t RC = 64;                    /* modules.mojo:59 */
    const int64_t n_chunks = (rows + RC - 1) / RC;
    if (rows * h * d < (1 << 17) || nthreads <= 1) {
        rms_rows(x, gamma, out, 0, rows, h, d, sc);
    } else {
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
        for (int64_t w = 0; w < n_chunks; ++w) {
            const int64_t r1 = (w + 1) * RC < rows ? (w + 1) * RC : rows;
            rms_rows(x, gamma, out, w * RC, r1, h, d, sc);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                     */
/* ------------------------------------------------------------------------ */
int64_t orc_rope_freqs(int64_t head_dim, int64_t dim, double freq_lo,
                       double freq_hi, float* freqs) {
    /* modules/rope.mojo:33-37 (== sparse/attention/rope.mojo:35-39) */
    const int64_t freq_dim = head_dim / 2 / dim;
    for (int64_t j = 0; j < freq_dim; ++j) {
        const float e = (float)j / (float)freq_dim;
        freqs[j] = (float)freq_lo / powf((float)freq_hi, e);
    }
    return freq_dim;
}

static void phase_of_slot(const float* posr, int64_t slot, int64_t dim,
                          const float* freqs, int64_t freq_dim, float* c, float* s) {
    /* rope.mojo:51-60: slot < dim*freq_dim -> axis = slot / fd, j = slot % fd */
    *c = 1.0f;
    *s = 0.0f;
    if (slot < dim * freq_dim) {
        const int64_t axis = slot / freq_dim;
        const int64_t j = slot % freq_dim;
        const float angle = posr[axis] * freqs[j];
        *c = cosf(angle);
        *s = sinf(angle);
    }
}

int orc_rope_phases_from_positions(const float* pos, int64_t l, int64_t dim,
                                   int64_t head_dim, const float* freqs,
                                   int64_t freq_dim, float* phases) {
    const int64_t half = head_dim / 2;
    for (int64_t r = 0; r < l; ++r)
        for (int64_t slot = 0; slot < half; ++slot)
            phase_of_slot(pos + r * dim, slot, dim, freqs, freq_dim,
                          &phases[(r * half + slot) * 2], &phases[(r * half + slot) * 2 + 1]);
    return 0;
}

int orc_rope_phases_from_coords(const int32_t* coords, int64_t n, int64_t ncols,
                                int64_t dim, int64_t head_dim, const float* freqs,
                                int64_t freq_dim, float* phases) {
    /* sparse/attention/rope.mojo:48-66: angle = Float32(coords.at(r, axis+1)) * freqs[j] */
    if (ncols != dim + 1) return -1; /* rope.mojo:129-130 */
    const int64_t half = head_dim / 2;
    float posr[16];
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t a = 0; a < dim && a < 16; ++a) posr[a] = (float)coords[r * ncols + a + 1];
        for (int64_t slot = 0; slot < half; ++slot)
            phase_of_slot(posr, slot, dim, freqs, freq_dim,
                          &phases[(r * half + slot) * 2], &phases[(r * half + slot) * 2 + 1]);
    }
    return 0;
}

void orc_grid_positions(int64_t r, float* pos) {
    /* models/sparse_structure_flow.mojo:139-149 */
    int64_t l = 0;
    for (int64_t i = 0; i < r; ++i)
        for (int64_t j = 0; j < r; ++j)
            for (int64_t k = 0; k < r; ++k) {
                pos[l * 3] = (float)i;
                pos[l * 3 + 1] = (float)j;
                pos[l * 3 + 2] = (float)k;
                ++l;
            }
}

int orc_apply_rotary(const float* x, const float* phases, float* out,
                     int64_t n, int64_t l, int64_t h, int64_t d) {
    /* modules/rope.mojo:64-88 (scalar serial 4-deep loop) */
    const int64_t half = d / 2;
    for (int64_t b = 0; b < n; ++b)
        for (int64_t jl = 0; jl < l; ++jl)
            for (int64_t head = 0; head < h; ++head)
                for (int64_t p = 0; p < half; ++p) {
                    const int64_t base = ((b * l + jl) * h + head) * d + 2 * p;
                    const float re = x[base], im = x[base + 1];
                    const float c = phases[(jl * half + p) * 2];
                    const float s = phases[(jl * half + p) * 2 + 1];
                    out[base] = re * c - im * s;
                    out[base + 1] = re * s + im * c;
                }
    return 0;
}

static void rotate_rows(const float* fp, const float* pp, float* op,
                        int64_t r0, int64_t r1, int64_t h, int64_t d) {
    const int64_t half = d / 2;
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t pbase = r * half * 2;
        for (int64_t head = 0; head < h; ++head) {
            const int64_t base = (r * h + head) * d;
            for (int64_t i = 0; i < d; i += 2) { /* rope.mojo:103-117, per-pair formula */
                const float re = fp[base + i], im = fp[base + i + 1];
                const float c = pp[pbase + i], s = pp[pbase + i + 1];
                op[base + i] = re * c - im * s;
                op[base + i + 1] = re * s + im * c;
            }
        }
    }
}

int orc_rope_rotate(const float* feats, const float* phases, float* out,
                    int64_t n, int64_t h, int64_t d, int nthreads) {
    /* sparse/attention/rope.mojo:76-126 */
    const int64_t RC = 64;
    const int64_t n_chunks = (n + RC - 1) / RC;
    if (n * h * d < (1 << 17) || nthreads <= 1) {
        rotate_rows(feats, phases, out, 0, n, h, d);
    } else {
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
        for (int64_t w = 0; w < n_chunks; ++w) {
            const int64_t r1 = (w + 1) * RC < n ? (w + 1) * RC : n;
            rotate_rows(feats, phases, out, w * RC, r1, h, d);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* activation: modules/nn.mojo:564-647                                      */
/* ------------------------------------------------------------------------ */
static inline float act_one(float v, int kind) {
    switch (kind) {
        case 0: return v > 0 ? v : 0.0f;                                   /* relu nn.mojo:564 */
        case 1: return v / (1.0f + expf(-v));                              /* silu nn.mojo:568 */
        case 2: return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f)); /* gelu nn.mojo:572 */
        default: {                                                         /* gelu_tanh nn.mojo:576-579 */
            const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
            return 0.5f * v * (1.0f + tanhf(inner));
        }
    }
}

int orc_activation(const float* x, float* out, int64_t n, int kind, int nthreads) {
    if (kind < 0 || kind > 3) return -1;   /* nn.mojo:598-599 "unknown activation" */
    const int64_t CH = 1 << 15;            /* nn.mojo:594 */
    const int64_t n_chunks = (n + CH - 1) / CH;
    if (n < (1 << 17) || nthreads <= 1) {
        for (int64_t i = 0; i < n; ++i) out[i] = act_one(x[i], kind);
    } else {
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
        for (int64_t c = 0; c < n_chunks; ++c) {
            const int64_t hi = (c + 1) * CH < n ? (c + 1) * CH : n;
            for (int64_t i = c * CH; i < hi; ++i) out[i] = act_one(x[i], kind);
        }
    }
    return 0;
}

void orc_add_bias(const float* x, const float* bias, float* out, int64_t rows, int64_t c) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < c; ++i) out[r * c + i] = x[r * c + i] + bias[i];
}

/* ------------------------------------------------------------------------ */
/* _gate: modules/transformer/modulated.mojo:22-33                          */
/* ------------------------------------------------------------------------ */
void orc_gate(const float* x, const float* g, float* out, int64_t n, int64_t l, int64_t c) {
    for (int64_t b = 0; b < n; ++b)
        for (int64_t j = 0; j < l; ++j)
            for (int64_t ci = 0; ci < c; ++ci) {
                const int64_t idx = (b * l + j) * c + ci;
                out[idx] = x[idx] * g[b * c + ci];
            }
}

/* ------------------------------------------------------------------------ */
/* pack_q_z / pack_kv_z: gpu/attention.mojo:566-594, 634-662                 */
/* ------------------------------------------------------------------------ */
/* gpu/linear.mojo:108-160, 326-388: acc += a[k] * b[k, n] for k in order. The
 * weight is transposed once so the inner loop runs over n (independent
 * accumulators, each still summed in k order). */
void orc_linear(const float* a, const float* w, float* c, int64_t m, int64_t n, int64_t k, int nthreads) {
    float* wt = (float*)malloc((size_t)(n * k) * sizeof(float));
    if (wt == NULL) return;
    for (int64_t j = 0; j < n; ++j)
        for (int64_t kk = 0; kk < k; ++kk) wt[kk * n + j] = w[j * k + kk];
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t i = 0; i < m; ++i) {
        float* ci = c + i * n;
        for (int64_t j = 0; j < n; ++j) ci[j] = 0.0f;
        for (int64_t kk = 0; kk < k; ++kk) {
            const float av = a[i * k + kk];
            const float* wr = wt + kk * n;
            for (int64_t j = 0; j < n; ++j) ci[j] = ci[j] + av * wr[j];
        }
    }
    free(wt);
}

void orc_pack_q(const float* qkv, float* qh, int64_t l, int64_t h, int64_t d, int64_t mp, int64_t stride) {
    const float scale = 1.0f / sqrtf((float)d); /* attention.mojo:587 */
    for (int64_t z = 0; z < h; ++z)
        for (int64_t t = 0; t < mp; ++t) {
            float* dst = qh + (z * mp + t) * d;
            if (t < l) {
                const float* src = qkv + t * stride + z * d;
                for (int64_t e = 0; e < d; ++e) dst[e] = src[e] * scale;
            } else {
                for (int64_t e = 0; e < d; ++e) dst[e] = 0.0f;
            }
        }
}

void orc_pack_kv(const float* qkv, float* kt, float* vh, int64_t l, int64_t h, int64_t d, int64_t lp) {
    const int64_t hd = h * d;
    for (int64_t z = 0; z < h; ++z)
        for (int64_t t = 0; t < lp; ++t) {
            const int64_t kb = z * d * lp;
            float* vdst = vh + (z * lp + t) * d;
            for (int64_t e = 0; e < d; ++e) {
                if (t < l) { /* attention.mojo:652-656 */
                    kt[kb + e * lp + t] = qkv[t * 3 * hd + hd + z * d + e];
                    vdst[e] = qkv[t * 3 * hd + 2 * hd + z * d + e];
                } else {
                    kt[kb + e * lp + t] = 0.0f;
                    vdst[e] = 0.0f;
                }
            }
        }
}

/* ------------------------------------------------------------------------ */
/* FlowEulerSampler: samplers/flow_euler.mojo                                */
/* ------------------------------------------------------------------------ */
/* _v_to_xstart (flow_euler.mojo:68-70): _scaled(x_t, 1 - sigma_min) minus
 * _scaled(v, c), each _scaled one f32 product (_binop_scalar, 56-57). */
void orc_flow_v_to_xstart(const float* x, const float* v, float* out, int64_t n, double t, double sigma_min) {
    const float a = (float)(1.0 - sigma_min);
    const float c = (float)(sigma_min + (1.0 - sigma_min) * t);
    for (int64_t i = 0; i < n; ++i) {
        const float xa = x[i] * a;
        const float vc = v[i] * c;
        out[i] = xa - vc;
    }
}

/* _inference CFG combine (flow_euler.mojo:173-176) */
void orc_flow_cfg(const float* pos, const float* neg, float* out, int64_t n, double g) {
    const float gp = (float)g;
    const float gn = (float)(1.0 - g);
    for (int64_t i = 0; i < n; ++i) {
        const float p = pos[i] * gp;
        const float q = neg[i] * gn;
        out[i] = p + q;
    }
}

/* _rescale_pred (flow_euler.mojo:75-149), serial f32 sums as the reference */
void orc_flow_rescale(const float* x_t, const float* pred, const float* pred_pos, float* out, int64_t rows,
                      int64_t row_size, double t, double sigma_min, double guidance_rescale,
                      const int64_t* seg_offsets, int64_t nseg_offsets) {
    const int64_t n = rows * row_size;
    float* x0_pos = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    float* x0_cfg = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    orc_flow_v_to_xstart(x_t, pred_pos, x0_pos, n, t, sigma_min);
    orc_flow_v_to_xstart(x_t, pred, x0_cfg, n, t, sigma_min);
    const int varlen = nseg_offsets > 0;
    const int64_t nb = varlen ? nseg_offsets - 1 : rows;
    const float gr = (float)guidance_rescale;
    const float a = (float)(1.0 - sigma_min);
    const float cc = (float)(sigma_min + (1.0 - sigma_min) * t);
    for (int64_t i = 0; i < n; ++i) out[i] = 0.0f; /* Tensor[F32](shape) is zero-filled */
    for (int64_t b = 0; b < nb; ++b) {
        const int64_t lo = varlen ? seg_offsets[b] * row_size : b * row_size;
        const int64_t hi = varlen ? seg_offsets[b + 1] * row_size : (b + 1) * row_size;
        const int64_t m = hi - lo;
        if (m == 0) continue;
        float std_pos, std_cfg;
        if (varlen) { /* VarLenTensor.std: sqrt(mean(x^2) - mean(x)^2), 113-126 */
            float s1 = 0, s2 = 0, c1 = 0, c2 = 0;
            for (int64_t e = lo; e < hi; ++e) {
                s1 += x0_pos[e];
                s2 += x0_pos[e] * x0_pos[e];
                c1 += x0_cfg[e];
                c2 += x0_cfg[e] * x0_cfg[e];
            }
            const float mp = s1 / (float)m;
            const float mc = c1 / (float)m;
            std_pos = sqrtf(s2 / (float)m - mp * mp);
            std_cfg = sqrtf(c2 / (float)m - mc * mc);
        } else { /* unbiased two-pass, 127-143 */
            float s1 = 0, c1 = 0;
            for (int64_t e = lo; e < hi; ++e) {
                s1 += x0_pos[e];
                c1 += x0_cfg[e];
            }
            const float mp = s1 / (float)m;
            const float mc = c1 / (float)m;
            float vp = 0, vc = 0;
            for (int64_t e = lo; e < hi; ++e) {
                const float dp = x0_pos[e] - mp;
                const float dc = x0_cfg[e] - mc;
                vp += dp * dp;
                vc += dc * dc;
            }
            std_pos = sqrtf(vp / (float)(m - 1));
            std_cfg = sqrtf(vc / (float)(m - 1));
        }
        const float ratio = std_pos / std_cfg;
        for (int64_t e = lo; e < hi; ++e) { /* 144-148 */
            const float x0r = x0_cfg[e] * ratio;
            const float x0 = gr * x0r + (1.0f - gr) * x0_cfg[e];
            out[e] = (a * x_t[e] - x0) / cc;
        }
    }
    free(x0_pos);
    free(x0_cfg);
}

/* sample = x_t - (t - t_prev) * v (flow_euler.mojo:210) */
void orc_flow_step(const float* x, const float* v, float* out, int64_t n, double t, double t_prev) {
    const float dt = (float)(t - t_prev);
    for (int64_t i = 0; i < n; ++i) {
        const float vd = v[i] * dt;
        out[i] = x[i] - vd;
    }
}

/* ------------------------------------------------------------------------ */
/* TimestepEmbedder.timestep_embedding: models/sparse_structure_flow.mojo:60-76 */
/* ------------------------------------------------------------------------ */
void orc_timestep_embedding(const float* t, int64_t n, int64_t dim,
                            double max_period, float* out) {
    const int64_t half = dim / 2;
    const float neg_log = -(float)log(max_period);           /* :69 */
    memset(out, 0, (size_t)(n * dim) * sizeof(float));       /* odd-dim zero column */
    for (int64_t r = 0; r < n; ++r)
        for (int64_t j = 0; j < half; ++j) {
            const float freq = expf(neg_log * (float)j / (float)half); /* :72 */
            const float angle = t[r] * freq;
            out[r * dim + j] = cosf(angle);
            out[r * dim + half + j] = sinf(angle);
        }
}

/* ------------------------------------------------------------------------ */
/* IEEE binary16 / bfloat16 rounding (round to nearest even)                */
/* ------------------------------------------------------------------------ */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mag = x & 0x7FFFFFFFu;
    if (mag >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (mag > 0x7F800000u ? 0x200u : 0u));
    if (mag >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
    if (mag < 0x38800000u) {                                   /* subnormal half */
        if (mag < 0x33000000u) return (uint16_t)sign;          /* < half of min subnormal */
        const uint32_t e = mag >> 23;
        const uint32_t m = (mag & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;                       /* 14 - (e - 127) + 13 - 1 ... */
        /* value = m * 2^(e-150); half subnormal unit = 2^-24 -> q = m >> (126-e) */
        const uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        uint32_t res = q;
        if (rem > halfway || (rem == halfway && (q & 1u))) res += 1u;
        return (uint16_t)(sign | res);
    }
    /* normal: rebias exponent 127 -> 15, keep 10 mantissa bits, RNE */
    uint32_t res = ((mag >> 13) - ((127u - 15u) << 10));
    const uint32_t rem = mag & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (res & 1u))) res += 1u;
    return (uint16_t)(sign | res);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    const uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_round_f16(const float* x, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(orc_f32_to_f16(x[i]));
}

void orc_round_bf16(const float* x, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &x[i], 4);
        if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) {
            u |= 0x400000u; /* quiet nan */
        } else {
            u += 0x7FFFu + ((u >> 16) & 1u);
        }
        u &= 0xFFFF0000u;
        memcpy(&out[i], &u, 4);
    }
}
