// t2h.hpp — C++ host-side mirror of the reference's per-token operator
// interface over the C ABI of libt2h.so (t2h.h).
//
// The reference's host language is Mojo; this header keeps its operator
// names, argument meaning, value semantics (inputs borrowed, a fresh output
// tensor returned) and error texts (the reference's `raise Error("...")` is a
// thrown t2h::Error with the same message), on device tensors whose every
// op is a libt2h kernel:
//   nn::LayerNorm32            modules/nn.mojo:297-375
//   nn::modulate               modules/nn.mojo:660-689
//   nn::activation             modules/nn.mojo:588-647
//   nn::MultiHeadRMSNorm       sparse/attention/modules.mojo:37-102
//   nn::RotaryPositionEmbedder, nn::apply_rotary_embedding
//                              modules/rope.mojo:17-88
//   nn::gate (_gate)           modules/transformer/modulated.mojo:22-33
//   nn::TimestepEmbedder       models/sparse_structure_flow.mojo:40-80
//   sparse::VarLenTensor, sparse::SparseTensor
//                              sparse/basic.mojo:89-155, 296-339, 433-439
//   sparse::mod_shift_scale    sparse/transformer/modulated.mojo:60-65
//   sparse::Modulation         sparse/transformer/modulated.mojo:24-57
//   sparse::SparseRotaryPositionEmbedder
//                              sparse/attention/rope.mojo:20-134
//   block::pack_block_consts, block::cross_block_enqueue
//                              gpu/block.mojo:217-397 (const layout 255-289)
//   block::ModulatedCrossBlock modules/transformer/modulated.mojo:177-200,
//                              sparse/transformer/modulated.mojo:187-226
//   samplers::FlowEulerSampler samplers/flow_euler.mojo:62-264
//   gpu::linear, gpu::linear_gate_residual
//                              gpu/linear.mojo:535-560, 662-684; gpu/block.mojo:86-110
//   gpu::attn_pack, gpu::qkv_linear_pack
//                              gpu/attention.mojo:507-662, 983-1013
//
// Calls run on the default HIP stream and are ordered with each other; a
// host read (Tensor::to_host, the SparseTensor layout check) synchronises.
// Output tensors are allocated per call (hipMalloc), as the reference
// allocates a fresh Tensor per op; the device entry points of t2h.h are the
// allocation-free hot path. Link with -lt2h (and the HIP runtime).
#ifndef T2H_HPP
#define T2H_HPP

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "t2h.h"

namespace t2h {

// The reference's Error: thrown with its message text.
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void check(int32_t rc) {
    if (rc != T2H_OK) throw Error(t2h_last_error());
}

inline void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

enum DType : int32_t { F32 = T2H_F32, F16 = T2H_F16, BF16 = T2H_BF16 };

inline size_t dtype_size(DType d) { return d == F32 ? 4 : 2; }

namespace detail {

// f32 <-> f16 / bf16 storage, round to nearest even (host side).
inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
inline float bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
inline uint16_t f32_to_f16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   // >= 65520 rounds to inf
    if (a < 0x38800000u) {                                      // below 2^-14: subnormal
        float v;
        std::memcpy(&v, &a, 4);
        return (uint16_t)(sign | (uint32_t)std::nearbyint(v * 16777216.0f));   // units of 2^-24, ties to even
    }
    uint32_t h = ((((a >> 23) - 112u) << 10) | ((a & 0x7FFFFFu) >> 13));
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}
inline float f16_to_f32(uint16_t b) {
    const uint32_t sign = (uint32_t)(b & 0x8000u) << 16, e = (b >> 10) & 0x1Fu, m = b & 0x3FFu;
    uint32_t u;
    if (e == 0) {
        const float v = (float)m * (1.0f / 16777216.0f);
        std::memcpy(&u, &v, 4);
        u |= sign;
    } else if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline std::shared_ptr<void> device_alloc(size_t bytes) {
    void* p = nullptr;
    if (bytes > 0) check_hip(hipMalloc(&p, bytes), "hipMalloc");
    return std::shared_ptr<void>(p, [](void* q) {
        if (q != nullptr) (void)hipFree(q);
    });
}

inline int64_t product(const std::vector<int64_t>& s) {
    int64_t n = 1;
    for (int64_t d : s) n *= d;
    return n;
}

}  // namespace detail

// Row-major device tensor with the reference Tensor's shape helpers
// (sparse/tensor.mojo:122-135): rows() = shape[0], row_size() = the
// product of the other dims. Copies share storage; ops return new tensors.
class Tensor {
public:
    Tensor() = default;

    static Tensor empty(std::vector<int64_t> shape, DType dt = F32) {
        Tensor t;
        t.shape_ = std::move(shape);
        t.dtype_ = dt;
        t.buf_ = detail::device_alloc((size_t)detail::product(t.shape_) * dtype_size(dt));
        return t;
    }

    static Tensor zeros(std::vector<int64_t> shape, DType dt = F32) {
        Tensor t = empty(std::move(shape), dt);
        if (t.numel() > 0) check_hip(hipMemset(t.data(), 0, t.bytes()), "hipMemset");
        return t;
    }

    // f32 host values stored in `dt` (rounded to nearest even for f16/bf16).
    static Tensor from_host(const float* src, std::vector<int64_t> shape, DType dt = F32) {
        Tensor t = empty(std::move(shape), dt);
        const int64_t n = t.numel();
        if (n == 0) return t;
        if (dt == F32) {
            check_hip(hipMemcpy(t.data(), src, t.bytes(), hipMemcpyHostToDevice), "hipMemcpy");
        } else {
            std::vector<uint16_t> h((size_t)n);
            for (int64_t i = 0; i < n; ++i)
                h[(size_t)i] = dt == F16 ? detail::f32_to_f16(src[i]) : detail::f32_to_bf16(src[i]);
            check_hip(hipMemcpy(t.data(), h.data(), t.bytes(), hipMemcpyHostToDevice), "hipMemcpy");
        }
        return t;
    }

    // Tensor.from_values (sparse/tensor.mojo): shape + row-major values.
    static Tensor from_values(std::vector<int64_t> shape, const std::vector<float>& values, DType dt = F32) {
        if ((int64_t)values.size() != detail::product(shape)) throw Error("Tensor.from_values: size mismatch");
        return from_host(values.data(), std::move(shape), dt);
    }

    // The values as f32 (synchronises).
    std::vector<float> to_host() const {
        std::vector<float> out((size_t)numel());
        if (out.empty()) return out;
        if (dtype_ == F32) {
            check_hip(hipMemcpy(out.data(), data(), bytes(), hipMemcpyDeviceToHost), "hipMemcpy");
        } else {
            std::vector<uint16_t> h(out.size());
            check_hip(hipMemcpy(h.data(), data(), bytes(), hipMemcpyDeviceToHost), "hipMemcpy");
            for (size_t i = 0; i < h.size(); ++i)
                out[i] = dtype_ == F16 ? detail::f16_to_f32(h[i]) : detail::bf16_to_f32(h[i]);
        }
        return out;
    }

    // A new tensor with a copy of the values (the reference's Tensor.copy()).
    Tensor clone() const {
        Tensor t = empty(shape_, dtype_);
        if (numel() > 0) check_hip(hipMemcpy(t.data(), data(), bytes(), hipMemcpyDeviceToDevice), "hipMemcpy");
        return t;
    }

    // Same storage, another shape of the same size.
    Tensor reshape(std::vector<int64_t> shape) const {
        if (detail::product(shape) != numel()) throw Error("Tensor.reshape: size mismatch");
        Tensor t = *this;
        t.shape_ = std::move(shape);
        return t;
    }

    const std::vector<int64_t>& shape() const { return shape_; }
    int64_t dim(int i) const { return shape_[(size_t)(i < 0 ? (int)shape_.size() + i : i)]; }
    int ndim() const { return (int)shape_.size(); }
    int64_t numel() const { return detail::product(shape_); }
    int64_t rows() const { return shape_.empty() ? 1 : shape_[0]; }
    int64_t row_size() const { return rows() == 0 ? 0 : numel() / rows(); }
    size_t bytes() const { return (size_t)numel() * dtype_size(dtype_); }
    DType dtype() const { return dtype_; }
    void* data() const { return buf_.get(); }
    // false for a default-constructed Tensor (an absent optional argument)
    bool defined() const { return static_cast<bool>(buf_) || !shape_.empty(); }

private:
    std::shared_ptr<void> buf_;
    std::vector<int64_t> shape_;
    DType dtype_ = F32;
};

// int32 device matrix [rows, cols]: the reference's IntMatrix (sparse/tensor.mojo:59-70),
// used for SparseTensor coords (b, x, y, z).
class IntMatrix {
public:
    IntMatrix() = default;
    static IntMatrix from_host(const int32_t* src, int64_t rows, int64_t cols) {
        IntMatrix m;
        m.rows_ = rows;
        m.cols_ = cols;
        m.buf_ = detail::device_alloc((size_t)(rows * cols) * 4);
        if (rows * cols > 0)
            check_hip(hipMemcpy(m.data(), src, (size_t)(rows * cols) * 4, hipMemcpyHostToDevice), "hipMemcpy");
        return m;
    }
    std::vector<int32_t> to_host() const {
        std::vector<int32_t> out((size_t)(rows_ * cols_));
        if (!out.empty())
            check_hip(hipMemcpy(out.data(), data(), out.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy");
        return out;
    }
    int64_t rows() const { return rows_; }
    int64_t cols() const { return cols_; }
    int32_t* data() const { return static_cast<int32_t*>(buf_.get()); }

private:
    std::shared_ptr<void> buf_;
    int64_t rows_ = 0, cols_ = 0;
};

namespace detail {

inline std::vector<float> host_floats(const Tensor& t) {
    if (t.dtype() != F32) throw Error("expected a float32 tensor");
    return t.to_host();
}

inline const float* f32_ptr(const Tensor& t, const char* what) {
    if (t.dtype() != F32) throw Error(std::string(what) + ": parameters must be float32");
    return static_cast<const float*>(t.data());
}

}  // namespace detail

// ---- modules/nn.mojo ---------------------------------------------------------
namespace nn {

constexpr int ACT_RELU = T2H_ACT_RELU, ACT_SILU = T2H_ACT_SILU, ACT_GELU = T2H_ACT_GELU,
              ACT_GELU_TANH = T2H_ACT_GELU_TANH;   // modules/nn.mojo:582-585

// nn.LayerNorm over the last dim (modules/nn.mojo:297-369): eps 1e-5 and
// affine by default, weight ones and bias zeros.
struct LayerNorm32 {
    int64_t num_channels;
    float eps;
    bool affine;
    Tensor weight, bias;

    explicit LayerNorm32(int64_t channels, double eps_ = 1e-5, bool affine_ = true)
        : num_channels(channels), eps((float)eps_), affine(affine_) {
        std::vector<float> ones((size_t)channels, 1.0f);
        weight = Tensor::from_host(ones.data(), {channels});
        bias = Tensor::zeros({channels});
    }

    Tensor forward(const Tensor& x) const {
        if (x.ndim() == 0 || x.dim(-1) != num_channels) throw Error("LayerNorm32: last dim mismatch");
        const int64_t rows = x.numel() / num_channels;
        Tensor out = Tensor::empty(x.shape(), x.dtype());
        check(t2h_ln_modulate(x.data(), out.data(), rows, (int32_t)num_channels, x.dtype(), eps,
                              affine ? T2H_LN_AFFINE : T2H_LN_PLAIN, affine ? (const float*)weight.data() : nullptr,
                              affine ? (const float*)bias.data() : nullptr, 0, nullptr, 1, 0, nullptr));
        return out;
    }
};

// x * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1): x [N, L, C], shift and
// scale [N, C] (modules/nn.mojo:660-689). Bit-exact.
inline Tensor modulate(const Tensor& x, const Tensor& shift, const Tensor& scale) {
    if (x.ndim() != 3) throw Error("modulate: expected x [N, L, C]");
    const int64_t n = x.dim(0), l = x.dim(1), c = x.dim(2);
    if (shift.numel() != n * c || scale.numel() != n * c) throw Error("modulate: shift/scale shape mismatch");
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    check(t2h_modulate(x.data(), out.data(), n * l, (int32_t)c, x.dtype(), detail::f32_ptr(shift, "modulate"),
                       detail::f32_ptr(scale, "modulate"), 0, nullptr, (int32_t)n, l, nullptr));
    return out;
}

// Elementwise activation (modules/nn.mojo:588-647).
inline Tensor activation(const Tensor& x, int kind) {
    if (kind < ACT_RELU || kind > ACT_GELU_TANH) throw Error("unknown activation");
    const int64_t c = x.ndim() ? x.dim(-1) : 1;
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    check(t2h_activation(x.data(), out.data(), nullptr, c ? x.numel() / c : 0, (int32_t)c, x.dtype(), kind,
                         nullptr));
    return out;
}

// F.normalize(x, dim=-1) * gamma * sqrt(dim) over x [..., H, D]
// (sparse/attention/modules.mojo:37-102); gamma [H, D] starts at ones.
struct MultiHeadRMSNorm {
    int64_t dim, heads;
    Tensor gamma;

    MultiHeadRMSNorm(int64_t dim_, int64_t heads_) : dim(dim_), heads(heads_) {
        std::vector<float> ones((size_t)(dim_ * heads_), 1.0f);
        gamma = Tensor::from_host(ones.data(), {heads_, dim_});
    }

    Tensor forward(const Tensor& x) const {
        if (x.ndim() < 2 || x.dim(-1) != dim || x.dim(-2) != heads)
            throw Error("MultiHeadRMSNorm: gamma shape mismatch");
        const int64_t rows = x.numel() / (dim * heads);
        Tensor out = Tensor::empty(x.shape(), x.dtype());
        check(t2h_qk_rmsnorm_rope(x.data(), nullptr, out.data(), nullptr, rows, 0, 0, (int32_t)heads, (int32_t)dim,
                                  x.dtype(), nullptr, nullptr, detail::f32_ptr(gamma, "MultiHeadRMSNorm"), nullptr,
                                  0, nullptr, 0, 3, nullptr, 0, nullptr, 0, 0, nullptr));
        return out;
    }
};

// freqs = freq_lo / freq_hi ** (arange(freq_dim) / freq_dim), f32
// (modules/rope.mojo:33-37).
inline std::vector<float> rope_freqs(int64_t head_dim, int64_t dim = 3, double freq_lo = 1.0,
                                     double freq_hi = 10000.0) {
    std::vector<float> f((size_t)(head_dim / 2 > 0 ? head_dim / 2 : 1));
    const int32_t fd = t2h_rope_freqs((int32_t)head_dim, (int32_t)dim, freq_lo, freq_hi, f.data(), (int32_t)f.size());
    if (fd < 0) check(fd);
    f.resize((size_t)fd);
    return f;
}

// Dense-path RoPE (modules/rope.mojo:17-61): forward(positions f32 [L, dim])
// -> phases [L, head_dim/2, 2] (cos, sin); axis-major slots, unit pad slots.
struct RotaryPositionEmbedder {
    int64_t head_dim, dim, freq_dim;
    std::vector<float> freqs;

    explicit RotaryPositionEmbedder(int64_t head_dim_, int64_t dim_ = 3, double freq_lo = 1.0,
                                    double freq_hi = 10000.0)
        : head_dim(head_dim_), dim(dim_) {
        if (head_dim_ % 2 != 0) throw Error("RotaryPositionEmbedder: head_dim must be even");
        freq_dim = head_dim_ / 2 / dim_;
        freqs = rope_freqs(head_dim_, dim_, freq_lo, freq_hi);
    }

    Tensor forward(const Tensor& positions) const {
        if (positions.ndim() != 2 || positions.dim(1) != dim)
            throw Error("RotaryPositionEmbedder: last dim of positions must be dim");
        const int64_t l = positions.dim(0);
        Tensor out = Tensor::empty({l, head_dim / 2, 2});
        check(t2h_rope_phases(static_cast<float*>(out.data()), l, (int32_t)head_dim, freqs.data(),
                              (int32_t)freqs.size(), (int32_t)dim, detail::f32_ptr(positions, "positions"), nullptr,
                              0, 0, nullptr));
        return out;
    }
};

// x [N, L, H, D] (adjacent re/im pairs), phases [L, D/2, 2] broadcast over N
// and H (modules/rope.mojo:64-88).
inline Tensor apply_rotary_embedding(const Tensor& x, const Tensor& phases) {
    if (x.ndim() != 4) throw Error("apply_rotary_embedding: expected [N, L, H, D]");
    const int64_t n = x.dim(0), l = x.dim(1), h = x.dim(2), d = x.dim(3);
    if (phases.ndim() != 3 || phases.dim(0) != l || phases.dim(1) != d / 2)
        throw Error("apply_rotary_embedding: phases shape mismatch");
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    // no RMS and no frequency table: the phases are the position source
    check(t2h_qk_rmsnorm_rope(x.data(), nullptr, out.data(), nullptr, n * l, 0, 0, (int32_t)h, (int32_t)d, x.dtype(),
                              nullptr, nullptr, nullptr, nullptr, 1, nullptr, 0, 3,
                              detail::f32_ptr(phases, "phases"), l, nullptr, 0, 0, nullptr));
    return out;
}

// x [N, L, C] * g [N, C] broadcast over L (modules/transformer/modulated.mojo:22-33).
inline Tensor gate(const Tensor& x, const Tensor& g) {
    if (x.ndim() != 3) throw Error("_gate: expected x [N, L, C]");
    const int64_t n = x.dim(0), l = x.dim(1), c = x.dim(2);
    if (g.numel() != n * c) throw Error("_gate: gate shape mismatch");
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    check(t2h_gate_residual(nullptr, x.data(), out.data(), nullptr, detail::f32_ptr(g, "_gate"), 0, n * l,
                            (int32_t)c, x.dtype(), nullptr, (int32_t)n, l, nullptr));
    return out;
}

// Sinusoidal timestep embedding (models/sparse_structure_flow.mojo:40-80);
// the MLP that follows it is a GEMM outside this path.
struct TimestepEmbedder {
    int64_t frequency_embedding_size;
    double max_period;

    explicit TimestepEmbedder(int64_t size = 256, double max_period_ = 10000.0)
        : frequency_embedding_size(size), max_period(max_period_) {}

    // t [N] f32 -> [N, frequency_embedding_size] f32
    Tensor timestep_embedding(const Tensor& t) const {
        const int64_t n = t.numel();
        Tensor out = Tensor::empty({n, frequency_embedding_size});
        check(t2h_timestep_embedding(detail::f32_ptr(t, "timestep_embedding"), out.data(), n,
                                     (int32_t)frequency_embedding_size, T2H_F32, max_period, nullptr));
        return out;
    }
};

}  // namespace nn

// ---- sparse/basic.mojo, sparse/transformer, sparse/attention ---------------------
namespace sparse {

constexpr int OP_ADD = T2H_OP_ADD, OP_SUB = T2H_OP_SUB, OP_MUL = T2H_OP_MUL,
              OP_DIV = T2H_OP_DIV;   // sparse/tensor.mojo:4-7

namespace detail {

inline std::shared_ptr<void> device_offsets(const std::vector<int64_t>& offsets) {
    auto p = t2h::detail::device_alloc(offsets.size() * 8);
    check_hip(hipMemcpy(p.get(), offsets.data(), offsets.size() * 8, hipMemcpyHostToDevice), "hipMemcpy");
    return p;
}

// feats [T, *] OP other[b(r)] with other [B, row] or [B, 1]
inline Tensor binop_rows(const Tensor& feats, const Tensor& other, int op, const int64_t* dev_offsets,
                         int64_t nbatch) {
    const int64_t rows = feats.rows(), c = feats.row_size();
    const int64_t oc = other.rows() ? other.numel() / other.rows() : 0;
    if (other.dtype() != F32) throw Error("elemwise_batch: other must be float32");
    Tensor out = Tensor::empty(feats.shape(), feats.dtype());
    check(t2h_binop_rows(feats.data(), static_cast<const float*>(other.data()), out.data(), rows, (int32_t)c,
                         (int32_t)oc, feats.dtype(), op, dev_offsets, (int32_t)nbatch, 0, nullptr));
    return out;
}

}  // namespace detail

// feats [T, *tail] with host offsets [B+1]: batch b owns rows
// [offsets[b], offsets[b+1]) (sparse/basic.mojo:89-247).
class VarLenTensor {
public:
    Tensor feats;
    std::vector<int64_t> offsets;

    VarLenTensor(Tensor f, std::vector<int64_t> offs) : feats(std::move(f)), offsets(std::move(offs)) {
        bool ok = !offsets.empty() && offsets[0] == 0 && offsets.back() == feats.rows();
        for (size_t i = 1; ok && i < offsets.size(); ++i) ok = offsets[i] >= offsets[i - 1];
        if (!ok) throw Error("VarLenTensor: invalid offsets");
        dev_ = detail::device_offsets(offsets);
    }

    int64_t batch_size() const { return (int64_t)offsets.size() - 1; }
    int64_t seqlen(int64_t b) const { return offsets[(size_t)b + 1] - offsets[(size_t)b]; }
    std::vector<int64_t> shape() const {
        std::vector<int64_t> s{batch_size()};
        s.insert(s.end(), feats.shape().begin() + 1, feats.shape().end());
        return s;
    }
    // row -> batch (sparse/basic.mojo:149-155)
    std::vector<int64_t> batch_broadcast_map() const {
        std::vector<int64_t> m;
        for (int64_t b = 0; b < batch_size(); ++b)
            for (int64_t i = 0; i < seqlen(b); ++i) m.push_back(b);
        return m;
    }
    VarLenTensor replace(Tensor f) const {
        if (f.rows() != feats.rows()) throw Error("VarLenTensor.replace: row count mismatch");
        VarLenTensor v = *this;
        v.feats = std::move(f);
        return v;
    }
    // feats[r] OP other[b(r)] (sparse/basic.mojo:204-207)
    VarLenTensor elemwise_batch(const Tensor& other, int op) const {
        if (other.rows() != batch_size()) throw Error("VarLenTensor.elemwise_batch: batch size mismatch");
        return replace(detail::binop_rows(feats, other, op, static_cast<const int64_t*>(dev_.get()), batch_size()));
    }
    // feats OP value, or value OP feats when reverse (sparse/tensor.mojo:200-203)
    VarLenTensor elemwise_scalar(float value, int op, bool reverse = false) const {
        const Tensor v = Tensor::from_host(&value, {1, 1});
        int o = op;
        if (reverse && op == OP_SUB) o = T2H_OP_RSUB;
        if (reverse && op == OP_DIV) o = T2H_OP_RDIV;
        return replace(detail::binop_rows(feats, v, o, nullptr, 1));
    }
    VarLenTensor operator+(const VarLenTensor& o) const {
        if (o.feats.numel() != feats.numel() || o.feats.dtype() != feats.dtype())
            throw Error("Tensor binop: size mismatch");
        Tensor out = Tensor::empty(feats.shape(), feats.dtype());
        check(t2h_gate_residual(feats.data(), o.feats.data(), out.data(), nullptr, nullptr, 0, feats.rows(),
                                (int32_t)feats.row_size(), feats.dtype(), nullptr, 1, 0, nullptr));
        return replace(out);
    }
    VarLenTensor operator+(float v) const { return elemwise_scalar(v, OP_ADD); }
    VarLenTensor operator-(float v) const { return elemwise_scalar(v, OP_SUB); }
    VarLenTensor operator*(float v) const { return elemwise_scalar(v, OP_MUL); }
    VarLenTensor operator/(float v) const { return elemwise_scalar(v, OP_DIV); }
    VarLenTensor operator-() const { return elemwise_scalar(-1.0f, OP_MUL); }

    const int64_t* device_offsets() const { return static_cast<const int64_t*>(dev_.get()); }

private:
    std::shared_ptr<void> dev_;
};

// feats [N, *tail] + int32 coords [N, 4] = (batch, x, y, z); the rows of a
// batch contiguous and batches ordered. The offsets are computed on the
// device from coords[:, 0] (sparse/basic.mojo:321-339) and checked on the
// host, with the reference's two errors.
class SparseTensor {
public:
    Tensor feats;
    IntMatrix coords;

    SparseTensor(Tensor f, IntMatrix c, int64_t batch_size = -1) : feats(std::move(f)), coords(std::move(c)) {
        if (feats.rows() != coords.rows()) throw Error("SparseTensor: feats/coords row mismatch");
        int64_t b = batch_size;
        if (b < 0) {   // IntMatrix.col_max(0) + 1
            if (coords.rows() == 0) throw Error("IntMatrix.col_max: empty matrix");
            const std::vector<int32_t> h = coords.to_host();
            int32_t mx = h[0];
            for (int64_t r = 0; r < coords.rows(); ++r) mx = h[(size_t)(r * coords.cols())] > mx ? h[(size_t)(r * coords.cols())] : mx;
            b = (int64_t)mx + 1;
        }
        batch_ = b;
        dev_ = t2h::detail::device_alloc((size_t)(b + 2) * 8);   // offsets [B+1] + the first-bad flag
        int64_t* off = static_cast<int64_t*>(dev_.get());
        check(t2h_coords_to_offsets(coords.data(), coords.rows(), (int32_t)coords.cols(), (int32_t)b, off, off + b + 1,
                                    nullptr));
        std::vector<int64_t> h((size_t)(b + 2));
        check_hip(hipMemcpy(h.data(), off, h.size() * 8, hipMemcpyDeviceToHost), "hipMemcpy");
        const int64_t bad = h[(size_t)b + 1];
        if (bad != INT64_MAX) {
            if (bad & 1) throw Error("SparseTensor: batch index out of range");
            throw Error("SparseTensor: batches must be ordered/contiguous");
        }
        offsets_.assign(h.begin(), h.begin() + b + 1);
    }

    int64_t batch_size() const { return batch_; }
    int64_t seqlen(int64_t b) const { return offsets_[(size_t)b + 1] - offsets_[(size_t)b]; }
    const std::vector<int64_t>& offsets() const { return offsets_; }
    const int64_t* device_offsets() const { return static_cast<const int64_t*>(dev_.get()); }

    SparseTensor replace(Tensor f) const {
        if (f.rows() != feats.rows()) throw Error("VarLenTensor.replace: row count mismatch");
        SparseTensor s = *this;
        s.feats = std::move(f);
        return s;
    }
    // the reference's x.vl
    VarLenTensor vl() const { return VarLenTensor(feats, offsets_); }

    // feats[r] OP other[b(r)] (sparse/basic.mojo:433-436)
    SparseTensor elemwise_batch(const Tensor& other, int op) const {
        if (other.rows() != batch_) throw Error("SparseTensor.elemwise_batch: batch size mismatch");
        return replace(detail::binop_rows(feats, other, op, device_offsets(), batch_));
    }
    // elementwise feats add (sparse/basic.mojo:438-439)
    SparseTensor operator+(const SparseTensor& o) const {
        if (o.feats.numel() != feats.numel() || o.feats.dtype() != feats.dtype())
            throw Error("Tensor binop: size mismatch");
        Tensor out = Tensor::empty(feats.shape(), feats.dtype());
        check(t2h_gate_residual(feats.data(), o.feats.data(), out.data(), nullptr, nullptr, 0, feats.rows(),
                                (int32_t)feats.row_size(), feats.dtype(), nullptr, 1, 0, nullptr));
        return replace(out);
    }

private:
    int64_t batch_ = 0;
    std::vector<int64_t> offsets_;
    std::shared_ptr<void> dev_;
};

// h * (1 + scale) + shift with [B, C] batch broadcast (sparse/transformer/modulated.mojo:60-65).
inline SparseTensor mod_shift_scale(const SparseTensor& h, const Tensor& shift, const Tensor& scale) {
    if (shift.rows() != h.batch_size() || scale.rows() != h.batch_size())
        throw Error("SparseTensor.elemwise_batch: batch size mismatch");
    const int64_t c = h.feats.row_size();
    Tensor out = Tensor::empty(h.feats.shape(), h.feats.dtype());
    check(t2h_modulate(h.feats.data(), out.data(), h.feats.rows(), (int32_t)c, h.feats.dtype(),
                       t2h::detail::f32_ptr(shift, "_mod_shift_scale"), t2h::detail::f32_ptr(scale, "_mod_shift_scale"),
                       0, h.device_offsets(), (int32_t)h.batch_size(), 0, nullptr));
    return h.replace(out);
}

// Modulation.chunks, share_mod branch (sparse/transformer/modulated.mojo:24-57):
// m = mod [N, 6C] + modulation [6C] row-broadcast, returned as the six [N, C]
// chunks shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp.
struct Modulation {
    Tensor modulation;   // [6C] f32

    explicit Modulation(Tensor m) : modulation(std::move(m)) {}

    std::vector<Tensor> chunks(const Tensor& mod, int64_t channels) const {
        if (mod.ndim() != 2 || mod.dim(1) != 6 * channels || modulation.numel() != 6 * channels)
            throw Error("Modulation: expected [N, 6C] modulation rows");
        const int64_t n = mod.dim(0);
        Tensor m = Tensor::empty({n, 6 * channels});
        check(t2h_modulation_add(t2h::detail::f32_ptr(mod, "Modulation"), t2h::detail::f32_ptr(modulation, "Modulation"),
                                 static_cast<float*>(m.data()), n, 6 * channels, nullptr));
        std::vector<Tensor> out;
        for (int64_t i = 0; i < 6; ++i) {   // slice_dim(1, i*C, (i+1)*C): a fresh [N, C] tensor
            Tensor t = Tensor::empty({n, channels});
            if (n > 0)
                check_hip(hipMemcpy2D(t.data(), (size_t)channels * 4, static_cast<float*>(m.data()) + i * channels,
                                      (size_t)(6 * channels) * 4, (size_t)channels * 4, (size_t)n,
                                      hipMemcpyDeviceToDevice),
                          "hipMemcpy2D");
            out.push_back(t);
        }
        return out;
    }
};

// RoPE from int voxel coords (sparse/attention/rope.mojo:20-134): embed
// rotates q and k (feats [N, H, head_dim]) in one kernel, the phases coming
// from each row's coords.
struct SparseRotaryPositionEmbedder {
    int64_t head_dim, dim, freq_dim;
    std::vector<float> freqs;

    explicit SparseRotaryPositionEmbedder(int64_t head_dim_, int64_t dim_ = 3, double freq_lo = 1.0,
                                          double freq_hi = 10000.0)
        : head_dim(head_dim_), dim(dim_) {
        if (head_dim_ % 2 != 0) throw Error("SparseRotaryPositionEmbedder: head_dim must be even");
        freq_dim = head_dim_ / 2 / dim_;
        freqs = nn::rope_freqs(head_dim_, dim_, freq_lo, freq_hi);
    }

    // _compute_phases: [N, head_dim/2, 2] (sparse/attention/rope.mojo:48-66)
    Tensor compute_phases(const SparseTensor& x) const {
        if (x.coords.cols() != dim + 1) throw Error("rope: coords must have dim+1 columns");
        Tensor out = Tensor::empty({x.coords.rows(), head_dim / 2, 2});
        check(t2h_rope_phases(static_cast<float*>(out.data()), x.coords.rows(), (int32_t)head_dim, freqs.data(),
                              (int32_t)freqs.size(), (int32_t)dim, nullptr, x.coords.data(), (int32_t)x.coords.cols(),
                              0, nullptr));
        return out;
    }

    std::pair<SparseTensor, SparseTensor> embed(const SparseTensor& q, const SparseTensor& k) const {
        if (q.coords.cols() != dim + 1) throw Error("rope: coords must have dim+1 columns");
        if (q.feats.dim(-1) != head_dim || k.feats.dim(-1) != head_dim) throw Error("rope: feats last dim != head_dim");
        if (q.feats.numel() != k.feats.numel() || q.feats.dtype() != k.feats.dtype())
            throw Error("rope: q/k shape mismatch");
        const int64_t rows = q.feats.rows();
        const int64_t heads = q.feats.row_size() / head_dim;
        Tensor qo = Tensor::empty(q.feats.shape(), q.feats.dtype());
        Tensor ko = Tensor::empty(k.feats.shape(), k.feats.dtype());
        check(t2h_qk_rmsnorm_rope(q.feats.data(), k.feats.data(), qo.data(), ko.data(), rows, 0, 0, (int32_t)heads,
                                  (int32_t)head_dim, q.feats.dtype(), nullptr, nullptr, nullptr, nullptr, 1,
                                  freqs.data(), (int32_t)freqs.size(), (int32_t)dim, nullptr, 0, q.coords.data(),
                                  (int32_t)q.coords.cols(), 0, nullptr));
        return {q.replace(qo), k.replace(ko)};
    }
};

}  // namespace sparse

// ---- the device-resident chain's GEMM and attention operands: gpu/linear.mojo,
// gpu/attention.mojo
namespace gpu {

namespace detail {

inline const float* opt_f32(const Tensor& t, int64_t n, const char* what) {
    if (!t.defined()) return nullptr;
    if (t.dtype() != F32 || t.numel() != n)
        throw Error(std::string(what) + ": must be " + std::to_string(n) + " float32 values");
    return static_cast<const float*>(t.data());
}

inline void check_gemm(const Tensor& x, const Tensor& w, const char* what) {
    if (x.ndim() != 2 || w.ndim() != 2 || x.dim(1) != w.dim(1) || x.dtype() != w.dtype() || x.dtype() == F32)
        throw Error(std::string(what) + ": x [rows, K] and weight [N, K] must be float16 or bfloat16 alike");
}

}  // namespace detail

// act(x @ weight^T + bias) on the matrix cores: GpuLinear.enqueue_gemm
// (gpu/linear.mojo:535-560) with the bias and activation in the store (the
// MLP's first linear + gelu_tanh_bias, 662-684). x [rows, K], weight [N, K]
// in the checkpoint layout, both f16 or both bf16; bias [N] f32 or absent;
// act a T2H_ACT_* kind or T2H_ACT_NONE; the output in out_dtype (F32 or x's).
inline Tensor linear(const Tensor& x, const Tensor& weight, const Tensor& bias = Tensor(), int act = T2H_ACT_NONE,
                     DType out_dtype = F32) {
    detail::check_gemm(x, weight, "linear");
    const int64_t rows = x.dim(0), k = x.dim(1), n = weight.dim(0);
    Tensor out = Tensor::empty({rows, n}, out_dtype);
    check(t2h_linear(x.data(), k, weight.data(), detail::opt_f32(bias, n, "linear: bias"), out.data(), n, rows,
                     (int32_t)k, (int32_t)n, x.dtype(), out_dtype, act, nullptr));
    return out;
}

// res + fl(fl(x @ weight^T + bias) * gate[b(r)]): an out-linear with the
// block's gated residual join in its store (gpu/block.mojo:86-110;
// sparse/transformer/modulated.mojo:214-226 for per-batch gate rows). gate
// [B, N] or [N] f32, or absent (res + fl(acc + bias)); the batch map as in
// t2h.h (offsets: device [B+1], or rows_per_batch). Returns a new tensor of
// res's dtype (f32 or x's).
inline Tensor linear_gate_residual(const Tensor& x, const Tensor& weight, const Tensor& res,
                                   const Tensor& bias = Tensor(), const Tensor& gate = Tensor(),
                                   const int64_t* offsets = nullptr, int32_t nbatch = 1,
                                   int64_t rows_per_batch = 0) {
    detail::check_gemm(x, weight, "linear_gate_residual");
    const int64_t rows = x.dim(0), k = x.dim(1), n = weight.dim(0);
    if (res.ndim() != 2 || res.dim(0) != rows || res.dim(1) != n || (res.dtype() != F32 && res.dtype() != x.dtype()))
        throw Error("linear_gate_residual: res must be [rows, N] of x's dtype or float32");
    if (gate.defined() && (gate.dtype() != F32 || gate.numel() != (int64_t)nbatch * n))
        throw Error("linear_gate_residual: gate must be [B, N] float32");
    Tensor out = Tensor::empty(res.shape(), res.dtype());
    check(t2h_linear_gate_residual(x.data(), k, weight.data(), detail::opt_f32(bias, n, "linear_gate_residual: bias"),
                                   res.data(), out.data(), n, rows, (int32_t)k, (int32_t)n, x.dtype(), res.dtype(),
                                   gate.defined() ? static_cast<const float*>(gate.data()) : nullptr, n, offsets,
                                   nbatch, rows_per_batch, nullptr));
    return out;
}

// The attention operands of the self-attention chain (gpu/attention.mojo:
// 566-594 pack_q_z, 634-662 pack_kv_z): qh [H, mp, D] = q * 1/sqrt(D),
// k [H, D, lp] (the reference's transposed layout) or [H, lp, D] (row-major,
// the faster one on MI355X), vh [H, lp, D]; rows past the tokens are zero.
struct AttnOperands {
    Tensor qh, k, vh;
};

// RoPE for the pack: the frequency table (empty: no RoPE) and the position
// source, int32 voxel coords [rows, 1 + 3] or a dense grid of side grid_res.
struct Rope {
    std::vector<float> freqs;
    const IntMatrix* coords = nullptr;
    int32_t grid_res = 0;
};

namespace detail {

struct PackOut {
    AttnOperands o;
    int64_t mp, lp;
};

inline PackOut pack_outputs(int64_t rows, int64_t heads, int64_t d, DType dt, int64_t mp, int64_t lp, bool kt) {
    PackOut p;
    p.mp = mp ? mp : rows;
    p.lp = lp ? lp : rows;
    p.o.qh = Tensor::empty({heads, p.mp, d}, dt);
    p.o.k = kt ? Tensor::empty({heads, d, p.lp}, dt) : Tensor::empty({heads, p.lp, d}, dt);
    p.o.vh = Tensor::empty({heads, p.lp, d}, dt);
    return p;
}

}  // namespace detail

// bias_rms_rope_qkv + pack_q_z + pack_kv_z (gpu/attention.mojo:507-563,
// 566-594, 634-662; sequence 987-1013) in one pass over the qkv GEMM output
// [rows, 3 * H * D]: +bias (q, k, v), RMS q and k (gammas [H, D]; absent:
// no RMS), RoPE q and k, then the head-major pack.
inline AttnOperands attn_pack(const Tensor& qkv, int32_t heads, const Tensor& bias, const Tensor& gamma_q,
                              const Tensor& gamma_k, const Rope& rope = Rope(), int64_t mp = 0, int64_t lp = 0,
                              bool k_transposed = true) {
    if (qkv.ndim() != 2 || heads <= 0 || qkv.dim(1) % (3 * heads) != 0)
        throw Error("attn_pack: qkv must be [rows, 3 * H * D]");
    const int64_t rows = qkv.dim(0), hd = qkv.dim(1) / 3, d = hd / heads;
    const DType dt = qkv.dtype();
    detail::PackOut p = detail::pack_outputs(rows, heads, d, dt, mp, lp, k_transposed);
    const char* q = static_cast<const char*>(qkv.data());
    const size_t es = dtype_size(dt);
    const float* b = detail::opt_f32(bias, 3 * hd, "attn_pack: bias");
    check(t2h_attn_pack(q, q + hd * es, q + 2 * hd * es, 3 * hd, rows, heads, (int32_t)d, dt, b, b ? b + hd : nullptr,
                        b ? b + 2 * hd : nullptr, detail::opt_f32(gamma_q, hd, "attn_pack: gamma_q"),
                        detail::opt_f32(gamma_k, hd, "attn_pack: gamma_k"), rope.freqs.empty() ? 0 : 1,
                        rope.freqs.empty() ? nullptr : rope.freqs.data(), (int32_t)rope.freqs.size(), 3, nullptr, 0,
                        rope.coords ? rope.coords->data() : nullptr, rope.coords ? (int32_t)rope.coords->cols() : 0,
                        rope.grid_res, p.o.qh.data(), p.mp, p.o.k.data(), p.o.vh.data(), p.lp, k_transposed ? 1 : 0,
                        nullptr));
    return p.o;
}

// The qkv linear on the matrix cores with attn_pack's epilogue and pack in
// its store (gpu/attention.mojo:983-1013): x [rows, K], weight [3 * H * D, K]
// (f16 or bf16), bias [3 * H * D] f32 or absent; the [rows, 3C] GEMM output
// never reaches memory.
inline AttnOperands qkv_linear_pack(const Tensor& x, const Tensor& weight, int32_t heads, const Tensor& bias,
                                    const Tensor& gamma_q, const Tensor& gamma_k, const Rope& rope = Rope(),
                                    int64_t mp = 0, int64_t lp = 0, bool k_transposed = true) {
    detail::check_gemm(x, weight, "qkv_linear_pack");
    if (heads <= 0 || weight.dim(0) % (3 * heads) != 0)
        throw Error("qkv_linear_pack: weight rows must be 3 * heads * head_dim");
    const int64_t rows = x.dim(0), k = x.dim(1), hd = weight.dim(0) / 3, d = hd / heads;
    detail::PackOut p = detail::pack_outputs(rows, heads, d, x.dtype(), mp, lp, k_transposed);
    const float* b = detail::opt_f32(bias, 3 * hd, "qkv_linear_pack: bias");
    check(t2h_qkv_linear_pack(x.data(), k, weight.data(), rows, (int32_t)k, heads, (int32_t)d, x.dtype(), b,
                              b ? b + hd : nullptr, b ? b + 2 * hd : nullptr,
                              detail::opt_f32(gamma_q, hd, "qkv_linear_pack: gamma_q"),
                              detail::opt_f32(gamma_k, hd, "qkv_linear_pack: gamma_k"), rope.freqs.empty() ? 0 : 1,
                              rope.freqs.empty() ? nullptr : rope.freqs.data(), (int32_t)rope.freqs.size(), 3, nullptr,
                              0, rope.coords ? rope.coords->data() : nullptr,
                              rope.coords ? (int32_t)rope.coords->cols() : 0, rope.grid_res, p.o.qh.data(), p.mp,
                              p.o.k.data(), p.o.vh.data(), p.lp, k_transposed ? 1 : 0, nullptr));
    return p.o;
}

}  // namespace gpu

// ---- the cross block's per-token glue: gpu/block.mojo:217-397,
// modules/transformer/modulated.mojo:177-200, sparse/transformer/modulated.mojo:187-226
namespace block {

// A block's GEMM / attention work, outside this library: takes the normed
// rows [T, C] and returns a new tensor of the same shape and dtype.
using Chain = std::function<Tensor(const Tensor&)>;

// const-buffer pair offsets in units of C (gpu/block.mojo:255-262)
constexpr int BK_NORM1 = 0;        // shift1, scale1           (norm1 modulate)
constexpr int BK_SELF_JOIN = 2;    // self_out bias, gate1     (self residual join)
constexpr int BK_NORM2 = 4;        // norm2 weight, bias       (affine norm2)
constexpr int BK_CROSS_JOIN = 6;   // cross_out bias, 0        (ungated cross join)
constexpr int BK_NORM3 = 8;        // shift3, scale3           (norm3 modulate)
constexpr int BK_MLP_JOIN = 10;    // mlp2 bias, gate3         (mlp residual join)
constexpr int BK_FLOATS = 12;      // buffer size in units of C

// The block's glue consts [12C] f32 in the reference's layout
// (gpu/block.mojo:255-289). m = the six adaLN chunks of one batch row
// (shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp); an absent
// out bias (a default Tensor) is zeros, as in the reference.
inline Tensor pack_block_consts(const std::vector<Tensor>& m, const Tensor& norm2_weight, const Tensor& norm2_bias,
                                const Tensor& self_out_bias = Tensor(), const Tensor& cross_out_bias = Tensor(),
                                const Tensor& mlp2_bias = Tensor()) {
    if (m.size() != 6) throw Error("gpu_cross_block_enqueue: expected 6 mod chunks");
    const int64_t c = m[0].numel();
    const Tensor* parts[BK_FLOATS] = {&m[0], &m[1], &self_out_bias, &m[2], &norm2_weight, &norm2_bias,
                                      &cross_out_bias, nullptr, &m[3], &m[4], &mlp2_bias, &m[5]};
    Tensor bk = Tensor::zeros({BK_FLOATS * c});
    for (int i = 0; i < BK_FLOATS; ++i) {
        if (parts[i] == nullptr || !parts[i]->defined()) continue;
        if (parts[i]->numel() != c || parts[i]->dtype() != F32)
            throw Error("pack_block_consts: every part must be " + std::to_string(c) + " float32 values");
        check_hip(hipMemcpy(static_cast<float*>(bk.data()) + i * c, parts[i]->data(), (size_t)c * 4,
                            hipMemcpyDeviceToDevice),
                  "hipMemcpy");
    }
    return bk;
}

namespace detail {

inline Tensor chain_out(const Chain& chain, const Tensor& in, const Tensor& like, const char* what) {
    Tensor h = chain(in);
    if (h.shape() != like.shape() || h.dtype() != like.dtype())
        throw Error(std::string("cross_block_enqueue: ") + what + " chain returned a tensor of another shape or dtype");
    return h;
}

}  // namespace detail

// One block against the resident rows xs [rows, C], updated in place and
// returned, in the order of gpu/block.mojo:304-397:
//   hs = LN(xs)*(1+scale1)+shift1;        h = self_chain(hs)
//   xs += (h + self_out_bias) * gate1;    hs = LN(xs)*w2 + b2
//   h = cross_chain(hs);                  xs += h + cross_out_bias
//   hs = LN(xs)*(1+scale3)+shift3;        h = mlp_chain(hs)
//   xs += (h + mlp2_bias) * gate3
// The chains return their output without the out-linear bias, which the
// joins fold in, as the reference's do. fused: each join and the next norm
// in one pass (t2h_block_join_ln).
inline Tensor& cross_block_enqueue(Tensor& xs, const Tensor& bk, const Chain& self_chain, const Chain& cross_chain,
                                   const Chain& mlp_chain, bool fused = true) {
    if (xs.ndim() != 2) throw Error("cross_block_enqueue: xs must be [rows, C]");
    const int64_t rows = xs.dim(0), c = xs.dim(1);
    if (bk.numel() != BK_FLOATS * c || bk.dtype() != F32)
        throw Error("cross_block_enqueue: consts must hold " + std::to_string(BK_FLOATS * c) + " floats");
    const float* k = static_cast<const float*>(bk.data());
    const int32_t ci = (int32_t)c;
    const DType dt = xs.dtype();
    Tensor hs = Tensor::empty(xs.shape(), dt);
    check(t2h_ln_mod_rows(xs.data(), hs.data(), k, rows, ci, BK_NORM1 * ci, 1, dt, nullptr));
    Tensor h = detail::chain_out(self_chain, hs, xs, "self");
    if (h.data() == hs.data()) hs = Tensor::empty(xs.shape(), dt);   // the chain handed back its input
    if (fused) {
        check(t2h_block_join_ln(xs.data(), h.data(), hs.data(), k, rows, ci, BK_SELF_JOIN * ci, 1, BK_NORM2 * ci, 2,
                                dt, nullptr));
    } else {
        check(t2h_gate_add_bias_rows(xs.data(), h.data(), k, rows, ci, BK_SELF_JOIN * ci, 1, dt, nullptr));
        check(t2h_ln_mod_rows(xs.data(), hs.data(), k, rows, ci, BK_NORM2 * ci, 2, dt, nullptr));
    }
    h = detail::chain_out(cross_chain, hs, xs, "cross");
    if (h.data() == hs.data()) hs = Tensor::empty(xs.shape(), dt);
    if (fused) {
        check(t2h_block_join_ln(xs.data(), h.data(), hs.data(), k, rows, ci, BK_CROSS_JOIN * ci, 0, BK_NORM3 * ci, 1,
                                dt, nullptr));
    } else {
        check(t2h_gate_add_bias_rows(xs.data(), h.data(), k, rows, ci, BK_CROSS_JOIN * ci, 0, dt, nullptr));
        check(t2h_ln_mod_rows(xs.data(), hs.data(), k, rows, ci, BK_NORM3 * ci, 1, dt, nullptr));
    }
    h = detail::chain_out(mlp_chain, hs, xs, "mlp");
    check(t2h_gate_add_bias_rows(xs.data(), h.data(), k, rows, ci, BK_MLP_JOIN * ci, 1, dt, nullptr));
    return xs;
}

// The glue of ModulatedTransformerCrossBlock / ModulatedSparseTransformerCrossBlock:
// norm1 and norm3 non-affine, norm2 affine, all with eps (1e-6 in the DiT
// blocks, loaders.mojo:53-60). `modulation` is the share_mod parameter [6C]
// (Modulation), or absent when `mod` already holds the chunks [B, 6C]. The
// chains return complete outputs (bias included), as the reference's
// attention modules do; each row reads its batch's adaLN chunk in place.
class ModulatedCrossBlock {
public:
    ModulatedCrossBlock(int64_t channels, Tensor norm2_weight, Tensor norm2_bias, Tensor modulation = Tensor(),
                        double eps = 1e-6)
        : c_(channels), eps_((float)eps), w2_(std::move(norm2_weight)), b2_(std::move(norm2_bias)),
          modulation_(std::move(modulation)) {
        if (w2_.numel() != c_ || b2_.numel() != c_ || w2_.dtype() != F32 || b2_.dtype() != F32)
            throw Error("ModulatedCrossBlock: norm2 weight and bias must be [C] float32");
    }

    // dense x [N, L, C], mod [N, 6C] (or [N, C] with the share_mod parameter's 6C added)
    Tensor forward(const Tensor& x, const Tensor& mod, const Chain& self_attn, const Chain& cross_attn,
                   const Chain& mlp) const {
        if (x.ndim() != 3 || x.dim(2) != c_) throw Error("LayerNorm32: last dim mismatch");
        const Tensor m = chunks(mod);
        if (m.dim(0) != x.dim(0)) throw Error("modulate: shift/scale shape mismatch");
        const Tensor out = run(x.reshape({x.dim(0) * x.dim(1), c_}), m, nullptr, (int32_t)x.dim(0), x.dim(1),
                               self_attn, cross_attn, mlp);
        return out.reshape(x.shape());
    }

    // sparse feats [T, C], mod [B, 6C]
    sparse::SparseTensor forward(const sparse::SparseTensor& x, const Tensor& mod, const Chain& self_attn,
                                 const Chain& cross_attn, const Chain& mlp) const {
        if (x.feats.ndim() != 2 || x.feats.dim(1) != c_) throw Error("LayerNorm32: last dim mismatch");
        const Tensor m = chunks(mod);
        if (m.dim(0) != x.batch_size()) throw Error("SparseTensor.elemwise_batch: batch size mismatch");
        return x.replace(run(x.feats, m, x.device_offsets(), (int32_t)x.batch_size(), 0, self_attn, cross_attn, mlp));
    }

private:
    // mod [B, 6C] f32, plus the share_mod parameter when there is one
    // (sparse/transformer/modulated.mojo:41-48)
    Tensor chunks(const Tensor& mod) const {
        if (mod.ndim() != 2 || mod.dim(1) != 6 * c_ || mod.dtype() != F32)
            throw Error("ModulatedCrossBlock: mod must be [B, 6C] float32");
        if (!modulation_.defined()) return mod;
        Tensor m = Tensor::empty(mod.shape());
        check(t2h_modulation_add(static_cast<const float*>(mod.data()), t2h::detail::f32_ptr(modulation_, "Modulation"),
                                 static_cast<float*>(m.data()), mod.dim(0), 6 * c_, nullptr));
        return m;
    }

    Tensor run(const Tensor& feats, const Tensor& m6, const int64_t* offsets, int32_t nbatch, int64_t rows_per_batch,
               const Chain& self_attn, const Chain& cross_attn, const Chain& mlp) const {
        const int64_t rows = feats.dim(0), ps = 6 * c_;
        const int32_t ci = (int32_t)c_;
        const DType dt = feats.dtype();
        const float* m = static_cast<const float*>(m6.data());   // chunk i of batch b at m + b * 6C + i * C
        const float* w2 = static_cast<const float*>(w2_.data());
        const float* b2 = static_cast<const float*>(b2_.data());
        // h = modulate(norm1(x), shift_msa, scale_msa)
        Tensor h = Tensor::empty(feats.shape(), dt);
        check(t2h_ln_modulate(feats.data(), h.data(), rows, ci, dt, eps_, T2H_LN_MODULATE, m, m + c_, ps, offsets,
                              nbatch, rows_per_batch, nullptr));
        h = detail::chain_out(self_attn, h, feats, "self");
        // y = x + h * gate_msa;  h2 = norm2(y) (affine)
        Tensor y = Tensor::empty(feats.shape(), dt), h2 = Tensor::empty(feats.shape(), dt);
        check(t2h_gate_residual_ln_modulate(feats.data(), h.data(), y.data(), h2.data(), nullptr, m + 2 * c_, ps, eps_,
                                            T2H_LN_AFFINE, w2, b2, 0, rows, ci, dt, offsets, nbatch, rows_per_batch,
                                            nullptr));
        h2 = detail::chain_out(cross_attn, h2, feats, "cross");
        // y = y + h2;  h3 = modulate(norm3(y), shift_mlp, scale_mlp)
        Tensor h3 = Tensor::empty(feats.shape(), dt);
        check(t2h_gate_residual_ln_modulate(y.data(), h2.data(), y.data(), h3.data(), nullptr, nullptr, 0, eps_,
                                            T2H_LN_MODULATE, m + 3 * c_, m + 4 * c_, ps, rows, ci, dt, offsets, nbatch,
                                            rows_per_batch, nullptr));
        h3 = detail::chain_out(mlp, h3, feats, "mlp");
        // y = y + h3 * gate_mlp
        check(t2h_gate_residual(y.data(), h3.data(), y.data(), nullptr, m + 5 * c_, ps, rows, ci, dt, offsets, nbatch,
                                rows_per_batch, nullptr));
        return y;
    }

    int64_t c_;
    float eps_;
    Tensor w2_, b2_, modulation_;
};

}  // namespace block

// ---- samplers/flow_euler.mojo -------------------------------------------------------
namespace samplers {

constexpr int GUIDANCE_NONE = 0, GUIDANCE_CFG = 1, GUIDANCE_CFG_INTERVAL = 2;   // flow_euler.mojo:27-29

// The velocity model (the DiT, outside this library): model(x_t, t * 1000,
// use_neg_cond) returns a tensor of x_t's shape and dtype.
using Model = std::function<Tensor(const Tensor& x_t, double t1000, bool use_neg_cond)>;

// np.linspace(1, 0, steps + 1) rescaled: rescale_t*t / (1 + (rescale_t-1)*t)
// (flow_euler.mojo:195-198), in f64.
inline std::vector<double> t_schedule(int steps, double rescale_t) {
    std::vector<double> out;
    for (int i = 0; i <= steps; ++i) {
        const double t = 1.0 - (double)i / (double)steps;
        out.push_back(rescale_t * t / (1.0 + (rescale_t - 1.0) * t));
    }
    return out;
}

// The edict FlowEulerSampler.sample returns (flow_euler.mojo:44-53).
struct SampleResult {
    Tensor samples;
    std::vector<Tensor> pred_x_t, pred_x_0;
};

// FlowEulerSampler / FlowEulerCfgSampler / FlowEulerGuidanceIntervalSampler
// (flow_euler.mojo:62-264). The step schedule and the guidance decisions stay
// on the host in f64, as in the reference; each step's tensor math (CFG
// combine, CFG rescale, Euler update, x_0 prediction) is one
// t2h_flow_euler_step call. The rescale's workspace is kept between steps.
class FlowEulerSampler {
public:
    explicit FlowEulerSampler(double sigma_min) : sigma_min_(sigma_min) {}

    // One step: {x_prev, pred_x0} from the predictions (v_neg null: none).
    // seg_offsets: the varlen token segments (per-segment biased std in the
    // rescale); empty: one segment per row.
    std::pair<Tensor, Tensor> step(const Tensor& x_t, const Tensor& v_pos, const Tensor* v_neg, double t, double t_prev,
                                   double guidance_strength = 1.0, double guidance_rescale = 0.0,
                                   const std::vector<int64_t>& seg_offsets = {}) {
        if (v_pos.shape() != x_t.shape() || v_pos.dtype() != x_t.dtype() ||
            (v_neg != nullptr && (v_neg->shape() != x_t.shape() || v_neg->dtype() != x_t.dtype())))
            throw Error("FlowEulerSampler: predictions must match x_t");
        const int64_t rows = x_t.rows(), rs = x_t.row_size();
        Tensor x_prev = Tensor::empty(x_t.shape(), x_t.dtype()), x0 = Tensor::empty(x_t.shape(), x_t.dtype());
        void* ws = nullptr;
        int64_t ws_bytes = 0;
        if (v_neg != nullptr && guidance_rescale > 0.0) {
            const int64_t need = t2h_flow_euler_workspace(rows, rs, (int32_t)seg_offsets.size());
            if (need > ws_bytes_) {
                ws_ = t2h::detail::device_alloc((size_t)need);
                ws_bytes_ = need;
            }
            ws = ws_.get();
            ws_bytes = ws_bytes_;
        }
        check(t2h_flow_euler_step(x_t.data(), v_pos.data(), v_neg != nullptr ? v_neg->data() : nullptr, x_prev.data(),
                                  x0.data(), rows, rs, x_t.dtype(), t, t_prev, sigma_min_, guidance_strength,
                                  guidance_rescale, seg_offsets.empty() ? nullptr : seg_offsets.data(),
                                  (int32_t)seg_offsets.size(), ws, ws_bytes, nullptr));
        return {x_prev, x0};
    }

    SampleResult sample(const Model& model, const Tensor& noise, int steps = 50, double rescale_t = 1.0) {
        return sample_impl(model, noise, steps, rescale_t, GUIDANCE_NONE, 1.0, 0.0, 1.0, 0.0, {});
    }
    SampleResult sample_cfg(const Model& model, const Tensor& noise, int steps = 50, double rescale_t = 1.0,
                            double guidance_strength = 3.0, double guidance_rescale = 0.0,
                            const std::vector<int64_t>& seg_offsets = {}) {
        return sample_impl(model, noise, steps, rescale_t, GUIDANCE_CFG, guidance_strength, 0.0, 1.0,
                           guidance_rescale, seg_offsets);
    }
    SampleResult sample_cfg_interval(const Model& model, const Tensor& noise, int steps = 50, double rescale_t = 1.0,
                                     double guidance_strength = 3.0, double interval_lo = 0.0,
                                     double interval_hi = 1.0, double guidance_rescale = 0.0,
                                     const std::vector<int64_t>& seg_offsets = {}) {
        return sample_impl(model, noise, steps, rescale_t, GUIDANCE_CFG_INTERVAL, guidance_strength, interval_lo,
                           interval_hi, guidance_rescale, seg_offsets);
    }

private:
    // _sample_impl (flow_euler.mojo:183-214) with _inference's branches
    // (151-181): the negative branch is evaluated only when it is used.
    SampleResult sample_impl(const Model& model, const Tensor& noise, int steps, double rescale_t, int mode, double g,
                             double lo, double hi, double gr, const std::vector<int64_t>& seg_offsets) {
        Tensor x = noise.clone();
        const std::vector<double> ts = t_schedule(steps, rescale_t);
        SampleResult ret;
        for (int i = 0; i < steps; ++i) {
            const double t = ts[(size_t)i], tp = ts[(size_t)i + 1];
            bool use_cfg = mode == GUIDANCE_CFG;
            if (mode == GUIDANCE_CFG_INTERVAL) use_cfg = lo <= t && t <= hi;
            std::pair<Tensor, Tensor> r;
            if (!use_cfg || g == 1.0) {
                r = step(x, model(x, 1000.0 * t, false), nullptr, t, tp, 1.0, gr, seg_offsets);
            } else if (g == 0.0) {
                r = step(x, model(x, 1000.0 * t, true), nullptr, t, tp, 1.0, gr, seg_offsets);
            } else {
                const Tensor pos = model(x, 1000.0 * t, false);
                const Tensor neg = model(x, 1000.0 * t, true);
                r = step(x, pos, &neg, t, tp, g, gr, seg_offsets);
            }
            x = r.first;
            ret.pred_x_t.push_back(r.first);
            ret.pred_x_0.push_back(r.second);
        }
        ret.samples = x;
        return ret;
    }

    double sigma_min_;
    std::shared_ptr<void> ws_;
    int64_t ws_bytes_ = 0;
};

}  // namespace samplers
}  // namespace t2h

#endif  // T2H_HPP
