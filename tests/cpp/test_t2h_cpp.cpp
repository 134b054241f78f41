// Tests of the C++ operator interface (include/t2h.hpp) on the GPU.
//
// The hand-computed cases are those of the reference's
// tests/parity/test_sparse_basic.mojo (make_varlen 21-25, make_sparse 28-43,
// layout 47-59, elemwise 73-91, sparse layout 149-158, contiguity 161-171);
// the numeric ops are checked against the C oracle (liboracle.so, the CPU
// restatement of the reference) on seeded inputs, bit for bit where the op
// has no reduction or transcendental, else with
//   err = |got - want| / max(|want|, 1) <= 1e-5 (f32 storage), 2e-3 (f16).
//
// Usage: test_t2h_cpp [name-substring]   (exit status 0 = all passed)
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "t2h.hpp"

extern "C" {
#include "oracle.h"
}

using t2h::Error;
using t2h::IntMatrix;
using t2h::Tensor;
namespace nn = t2h::nn;
namespace sp = t2h::sparse;

namespace {

struct Failure {
    std::string what;
};

#define EXPECT(cond)                                                                  \
    do {                                                                              \
        if (!(cond)) throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond}; \
    } while (0)

std::vector<float> randn(uint64_t seed, int64_t n, double std = 1.0) {
    orc_rng r;
    orc_rng_init(&r, seed);
    std::vector<float> v((size_t)n);
    orc_randn(&r, v.data(), n, 0.0, std);
    return v;
}

std::vector<float> round_f16(const std::vector<float>& x) {
    std::vector<float> o(x.size());
    orc_round_f16(x.data(), o.data(), (int64_t)x.size());
    return o;
}

double max_err(const std::vector<float>& got, const std::vector<float>& want) {
    if (got.size() != want.size()) throw Failure{"size mismatch"};
    double m = 0.0;
    for (size_t i = 0; i < got.size(); ++i) {
        if (!std::isfinite(got[i])) return INFINITY;
        const double e = std::fabs((double)got[i] - want[i]) / std::fmax(std::fabs((double)want[i]), 1.0);
        m = e > m ? e : m;
    }
    return m;
}

void expect_close(const std::vector<float>& got, const std::vector<float>& want, double tol, const char* what) {
    const double e = max_err(got, want);
    std::printf("    %s: max err %.3e (tol %g)\n", what, e, tol);
    if (!(e <= tol)) throw Failure{std::string(what) + ": max err " + std::to_string(e)};
}

void expect_bits(const std::vector<float>& got, const std::vector<float>& want, const char* what) {
    if (got.size() != want.size() || std::memcmp(got.data(), want.data(), got.size() * 4) != 0)
        throw Failure{std::string(what) + ": not bit-exact"};
    std::printf("    %s: bit-exact (%zu values)\n", what, got.size());
}

template <class F>
void expect_error(F&& f, const char* text) {
    try {
        f();
    } catch (const Error& e) {
        if (std::strstr(e.what(), text) == nullptr)
            throw Failure{std::string("wrong error: '") + e.what() + "', expected '" + text + "'"};
        return;
    }
    throw Failure{std::string("no error raised, expected '") + text + "'"};
}

// ---- tests/parity/test_sparse_basic.mojo ------------------------------------------
sp::VarLenTensor make_varlen() {   // 21-25
    return sp::VarLenTensor(Tensor::from_values({5, 2}, {1, 2, 3, 4, 5, 6, 7, 8, 9, 10}), {0, 2, 5});
}

sp::SparseTensor make_sparse() {   // 28-43
    const int32_t c[5][4] = {{0, 0, 0, 0}, {0, 1, 0, 1}, {1, 0, 1, 0}, {1, 1, 1, 1}, {1, 1, 0, 0}};
    return sp::SparseTensor(Tensor::from_values({5, 2}, {1, 2, 3, 4, 5, 6, 7, 8, 9, 10}),
                            IntMatrix::from_host(&c[0][0], 5, 4));
}

void test_varlen_shape_and_layout() {   // 47-59
    const auto x = make_varlen();
    EXPECT(x.batch_size() == 2);
    EXPECT(x.shape()[0] == 2 && x.shape()[1] == 2);
    EXPECT(x.seqlen(0) == 2 && x.seqlen(1) == 3);
    const auto bm = x.batch_broadcast_map();
    EXPECT(bm[0] == 0 && bm[1] == 0 && bm[2] == 1 && bm[4] == 1);
    expect_error([] { sp::VarLenTensor(Tensor::zeros({5, 2}), {0, 3, 2, 5}); }, "VarLenTensor: invalid offsets");
}

void test_varlen_elemwise() {   // 73-91, plus the reverse scalar forms
    const auto x = make_varlen();
    const auto y = ((x + 1.0f) * 2.0f).feats.to_host();
    EXPECT(y[0] == 4.0f && y[9] == 22.0f);
    EXPECT((x + x).feats.to_host()[3] == 8.0f);
    EXPECT((-x).feats.to_host()[0] == -1.0f);
    const auto w = x.elemwise_batch(Tensor::from_values({2, 1}, {10, 100}), sp::OP_ADD).feats.to_host();
    EXPECT(w[0] == 11.0f && w[4] == 105.0f);
    const auto w2 = x.elemwise_batch(Tensor::from_values({2, 2}, {10, 20, 100, 200}), sp::OP_ADD).feats.to_host();
    EXPECT(w2[1] == 22.0f && w2[9] == 210.0f);
    const auto f = x.feats.to_host();
    for (int op = sp::OP_ADD; op <= sp::OP_DIV; ++op)
        for (int rev = 0; rev < 2; ++rev) {
            std::vector<float> want(f.size());
            orc_binop_scalar(f.data(), 3.0f, want.data(), (int64_t)f.size(), op, rev);
            expect_bits(x.elemwise_scalar(3.0f, op, rev != 0).feats.to_host(), want, "elemwise_scalar");
        }
    expect_error([&] { x.elemwise_batch(Tensor::zeros({3, 1}), sp::OP_ADD); }, "batch size mismatch");
}

void test_sparse_layout_from_coords() {   // 149-158
    const auto x = make_sparse();
    EXPECT(x.batch_size() == 2);
    EXPECT(x.seqlen(0) == 2 && x.seqlen(1) == 3);
    EXPECT((x.offsets() == std::vector<int64_t>{0, 2, 5}));
    const auto v = x.vl();
    EXPECT(v.batch_size() == 2 && v.seqlen(1) == 3);
}

void test_sparse_contiguity_enforced() {   // 161-171, and the out-of-range branch
    expect_error(
        [] {
            const int32_t c[2][4] = {{1, 0, 0, 0}, {0, 0, 0, 0}};   // batch 1 before batch 0
            sp::SparseTensor(Tensor::zeros({2, 1}), IntMatrix::from_host(&c[0][0], 2, 4));
        },
        "ordered/contiguous");
    expect_error(
        [] {
            const int32_t c[3][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {5, 0, 0, 0}};
            sp::SparseTensor(Tensor::zeros({3, 1}), IntMatrix::from_host(&c[0][0], 3, 4), 2);
        },
        "out of range");
    expect_error([] { sp::SparseTensor(Tensor::zeros({2, 1}), IntMatrix::from_host(nullptr, 0, 4)); },
                 "feats/coords row mismatch");
}

void test_sparse_elemwise_batch() {
    const auto x = make_sparse();
    const Tensor b = Tensor::from_values({2, 2}, {10, 20, 100, 200});
    const auto y = x.elemwise_batch(b, sp::OP_ADD).feats.to_host();
    EXPECT(y[0] == 11.0f && y[9] == 210.0f);
    EXPECT(x.elemwise_batch(b, sp::OP_MUL).feats.to_host()[1] == 40.0f);
    const auto s = x.elemwise_batch(Tensor::from_values({2, 1}, {10, 100}), sp::OP_ADD).feats.to_host();
    EXPECT(s[0] == 11.0f && s[4] == 105.0f);
    EXPECT((x + x).feats.to_host()[9] == 20.0f);
}

// ---- numeric parity against the oracle -------------------------------------------
void test_layernorm32() {
    const int64_t rows = 67, c = 1536;
    const auto x = randn(1, rows * c, 2.0);
    const auto w = randn(2, c, 0.5), b = randn(3, c, 0.5);
    for (t2h::DType dt : {t2h::F32, t2h::F16}) {
        const auto xin = dt == t2h::F32 ? x : round_f16(x);
        nn::LayerNorm32 ln(c);   // eps 1e-5, affine, weight ones / bias zeros
        std::vector<float> want((size_t)(rows * c));
        const std::vector<float> ones((size_t)c, 1.0f), zeros((size_t)c, 0.0f);
        orc_layernorm(xin.data(), want.data(), rows, c, 1e-5, 1, ones.data(), zeros.data());
        const Tensor xd = Tensor::from_host(x.data(), {rows, c}, dt);
        const double tol = dt == t2h::F32 ? 1e-5 : 2e-3;
        expect_close(ln.forward(xd).to_host(), want, tol, "LayerNorm32 default params");
        ln.weight = Tensor::from_host(w.data(), {c});
        ln.bias = Tensor::from_host(b.data(), {c});
        orc_layernorm(xin.data(), want.data(), rows, c, 1e-5, 1, w.data(), b.data());
        expect_close(ln.forward(xd).to_host(), want, tol, "LayerNorm32 affine");
        nn::LayerNorm32 plain(c, 1e-6, false);
        orc_layernorm(xin.data(), want.data(), rows, c, 1e-6, 0, nullptr, nullptr);
        expect_close(plain.forward(xd.reshape({1, rows, c})).to_host(), want, tol, "LayerNorm32 no affine");
    }
    expect_error([] { nn::LayerNorm32(8).forward(Tensor::zeros({2, 9})); }, "LayerNorm32: last dim mismatch");
}

void test_modulate_and_gate() {
    const int64_t n = 3, l = 41, c = 1024;
    const auto x = randn(4, n * l * c), sh = randn(5, n * c, 0.1), sc = randn(6, n * c, 0.1);
    const Tensor xd = Tensor::from_host(x.data(), {n, l, c});
    const Tensor shd = Tensor::from_host(sh.data(), {n, c}), scd = Tensor::from_host(sc.data(), {n, c});
    std::vector<float> want((size_t)(n * l * c));
    orc_modulate(x.data(), sh.data(), sc.data(), want.data(), n, l, c);
    expect_bits(nn::modulate(xd, shd, scd).to_host(), want, "modulate");
    orc_gate(x.data(), sc.data(), want.data(), n, l, c);
    expect_bits(nn::gate(xd, scd).to_host(), want, "_gate");
    expect_error([&] { nn::modulate(xd, Tensor::zeros({n, c - 1}), scd); }, "modulate: shift/scale shape mismatch");
}

void test_mod_shift_scale_sparse() {
    // three batches, the middle one empty
    const int64_t rows = 300, c = 1536;
    std::vector<int32_t> coords((size_t)rows * 4, 0);
    for (int64_t r = 0; r < rows; ++r) coords[(size_t)r * 4] = r < 120 ? 0 : 2;
    const auto x = randn(7, rows * c), sh = randn(8, 3 * c, 0.1), sc = randn(9, 3 * c, 0.1);
    const sp::SparseTensor h(Tensor::from_host(x.data(), {rows, c}), IntMatrix::from_host(coords.data(), rows, 4), 3);
    EXPECT((h.offsets() == std::vector<int64_t>{0, 120, 120, 300}));
    std::vector<int64_t> off(4);
    EXPECT(orc_cal_offsets(coords.data(), rows, 4, 3, off.data()) == 0);
    EXPECT(off == h.offsets());
    std::vector<float> want((size_t)(rows * c));
    orc_mod_shift_scale(x.data(), sh.data(), sc.data(), off.data(), 3, want.data(), rows, c);
    const auto got = sp::mod_shift_scale(h, Tensor::from_host(sh.data(), {3, c}), Tensor::from_host(sc.data(), {3, c}));
    expect_bits(got.feats.to_host(), want, "_mod_shift_scale");
    expect_error([&] { sp::mod_shift_scale(h, Tensor::zeros({2, c}), Tensor::zeros({2, c})); }, "batch size mismatch");
}

void test_activation() {
    const int64_t rows = 33, c = 1000;
    const auto x = randn(10, rows * c, 3.0);
    const Tensor xd = Tensor::from_host(x.data(), {rows, c});
    for (int kind : {nn::ACT_RELU, nn::ACT_SILU, nn::ACT_GELU, nn::ACT_GELU_TANH}) {
        std::vector<float> want(x.size());
        EXPECT(orc_activation(x.data(), want.data(), rows * c, kind, 1) == 0);
        expect_close(nn::activation(xd, kind).to_host(), want, 1e-5, "activation");
    }
    expect_error([&] { nn::activation(xd, 7); }, "unknown activation");
}

void test_multihead_rmsnorm_and_rope() {
    // MultiHeadRMSNorm then apply_rotary_embedding(x [N, L, H, D], phases) with
    // RotaryPositionEmbedder.forward(grid positions), the dense attention order
    const int64_t n = 2, res = 4, l = res * res * res, h = 12, d = 128;
    const auto q = randn(11, n * l * h * d), g = randn(12, h * d, 0.5);
    nn::MultiHeadRMSNorm rms(d, h);
    rms.gamma = Tensor::from_host(g.data(), {h, d});
    std::vector<float> pos((size_t)(l * 3));
    orc_grid_positions(res, pos.data());
    nn::RotaryPositionEmbedder emb(d);
    std::vector<float> freqs((size_t)(d / 2));
    const int64_t fd = orc_rope_freqs(d, 3, 1.0, 10000.0, freqs.data());
    EXPECT(fd == emb.freq_dim && (int64_t)emb.freqs.size() == fd);
    EXPECT(std::memcmp(freqs.data(), emb.freqs.data(), (size_t)fd * 4) == 0);
    std::vector<float> ph_want((size_t)(l * d));
    EXPECT(orc_rope_phases_from_positions(pos.data(), l, 3, d, freqs.data(), fd, ph_want.data()) == 0);
    const Tensor phases = emb.forward(Tensor::from_host(pos.data(), {l, 3}));
    expect_close(phases.to_host(), ph_want, 1e-5, "RotaryPositionEmbedder.forward");

    std::vector<float> normed(q.size()), want(q.size());
    EXPECT(orc_multihead_rmsnorm(q.data(), g.data(), normed.data(), n * l, h, d, 1) == 0);
    const Tensor qd = Tensor::from_host(q.data(), {n, l, h, d});
    const Tensor got_rms = rms.forward(qd);
    expect_close(got_rms.to_host(), normed, 1e-5, "MultiHeadRMSNorm");
    EXPECT(orc_apply_rotary(normed.data(), ph_want.data(), want.data(), n, l, h, d) == 0);
    expect_close(nn::apply_rotary_embedding(got_rms, phases).to_host(), want, 1e-5,
                 "MultiHeadRMSNorm + apply_rotary_embedding");
    expect_error([&] { nn::MultiHeadRMSNorm(64, h).forward(qd); }, "MultiHeadRMSNorm: gamma shape mismatch");
    expect_error([] { nn::RotaryPositionEmbedder(63); }, "head_dim must be even");
}

void test_sparse_rope_embed() {
    // SparseRotaryPositionEmbedder.embed(q, k) on voxel coords, f32 and f16
    const int64_t rows = 515, h = 12, d = 128, res = 64;
    std::vector<int32_t> coords((size_t)rows * 4);
    orc_rng r;
    orc_rng_init(&r, 13);
    for (int64_t i = 0; i < rows; ++i) {
        coords[(size_t)i * 4] = i < 200 ? 0 : 1;
        for (int a = 1; a < 4; ++a) coords[(size_t)i * 4 + a] = (int32_t)(orc_rng_next_u64(&r) % res);
    }
    const auto q = randn(14, rows * h * d), k = randn(15, rows * h * d);
    sp::SparseRotaryPositionEmbedder emb(d);
    std::vector<float> ph((size_t)(rows * d));
    EXPECT(orc_rope_phases_from_coords(coords.data(), rows, 4, 3, d, emb.freqs.data(), emb.freq_dim, ph.data()) == 0);
    const IntMatrix cm = IntMatrix::from_host(coords.data(), rows, 4);
    for (t2h::DType dt : {t2h::F32, t2h::F16}) {
        const auto qi = dt == t2h::F32 ? q : round_f16(q), ki = dt == t2h::F32 ? k : round_f16(k);
        const sp::SparseTensor sq(Tensor::from_host(q.data(), {rows, h, d}, dt), cm, 2);
        const sp::SparseTensor sk(Tensor::from_host(k.data(), {rows, h, d}, dt), cm, 2);
        if (dt == t2h::F32) expect_close(emb.compute_phases(sq).to_host(), ph, 1e-5, "_compute_phases");
        std::vector<float> wq(q.size()), wk(k.size());
        EXPECT(orc_rope_rotate(qi.data(), ph.data(), wq.data(), rows, h, d, 1) == 0);
        EXPECT(orc_rope_rotate(ki.data(), ph.data(), wk.data(), rows, h, d, 1) == 0);
        const auto qk = emb.embed(sq, sk);
        const double tol = dt == t2h::F32 ? 1e-5 : 2e-3;
        expect_close(qk.first.feats.to_host(), wq, tol, "embed q");
        expect_close(qk.second.feats.to_host(), wk, tol, "embed k");
    }
}

void test_timestep_embedder() {
    orc_rng r;
    orc_rng_init(&r, 501);
    std::vector<float> t(64);
    orc_uniform(&r, t.data(), 64, 0.0, 1.0);
    for (float& v : t) v *= 1000.0f;   // the pipeline passes t * 1000
    for (int64_t dim : {256, 255}) {
        nn::TimestepEmbedder te(dim);
        std::vector<float> want((size_t)(64 * dim));
        orc_timestep_embedding(t.data(), 64, dim, 10000.0, want.data());
        expect_close(te.timestep_embedding(Tensor::from_host(t.data(), {64})).to_host(), want, 1e-5,
                     "timestep_embedding");
    }
}

void test_modulation_chunks() {
    const int64_t n = 2, c = 1536;
    const auto mod = randn(16, n * 6 * c), par = randn(17, 6 * c, 0.02);
    sp::Modulation m(Tensor::from_host(par.data(), {6 * c}));
    const auto chunks = m.chunks(Tensor::from_host(mod.data(), {n, 6 * c}), c);
    EXPECT(chunks.size() == 6);
    std::vector<float> full((size_t)(n * 6 * c));
    orc_modulation_add(mod.data(), par.data(), full.data(), n, 6 * c);
    for (int64_t i = 0; i < 6; ++i) {
        std::vector<float> want((size_t)(n * c));
        for (int64_t b = 0; b < n; ++b)
            std::memcpy(&want[(size_t)(b * c)], &full[(size_t)(b * 6 * c + i * c)], (size_t)c * 4);
        expect_bits(chunks[(size_t)i].to_host(), want, "Modulation chunk");
    }
    expect_error([&] { m.chunks(Tensor::zeros({n, 5 * c}), c); }, "Modulation: expected [N, 6C] modulation rows");
}

// ---- the cross block's glue (modules/transformer/modulated.mojo:177-200,
// sparse/transformer/modulated.mojo:187-226, gpu/block.mojo:217-397) ---------------
namespace blk = t2h::block;

// Device chains built from bit-exact elementwise ops, so that the host side
// repeats them exactly: self h * 0.5, cross h + 0.25, mlp h * -0.75.
Tensor scaled(const Tensor& h, float v, int op) {
    const int64_t rows = h.rows();
    return sp::VarLenTensor(h, {0, rows}).elemwise_scalar(v, op).feats;
}
std::vector<float> host_scaled(const std::vector<float>& h, float v, int op) {
    std::vector<float> o(h.size());
    orc_binop_scalar(h.data(), v, o.data(), (int64_t)h.size(), op, 0);
    return o;
}

// host: LN (non-affine, or affine with w/b) over rows of c
std::vector<float> host_ln(const std::vector<float>& x, int64_t c, const float* w = nullptr, const float* b = nullptr) {
    std::vector<float> o(x.size());
    orc_layernorm(x.data(), o.data(), (int64_t)x.size() / c, c, 1e-6, w != nullptr, w, b);
    return o;
}
// host: fl(h * gate[b(r)]) added to x, with gate rows [B, C] and the batch offsets
std::vector<float> host_gated_add(const std::vector<float>& x, const std::vector<float>& h, const float* gate_rows,
                                  const std::vector<int64_t>& offsets, int64_t c) {
    const int64_t rows = (int64_t)x.size() / c, nb = (int64_t)offsets.size() - 1;
    std::vector<int64_t> map((size_t)rows);
    orc_batch_broadcast_map(offsets.data(), nb, map.data());
    std::vector<float> t(x.size()), o(x.size());
    orc_binop_rows(h.data(), gate_rows, map.data(), t.data(), rows, c, c, sp::OP_MUL);
    orc_binop_flat(x.data(), t.data(), o.data(), (int64_t)x.size(), sp::OP_ADD);
    return o;
}
// the rows of chunk i of a [B, 6C] modulation: [B, C]
std::vector<float> chunk_rows(const std::vector<float>& m6, int64_t nb, int64_t c, int i) {
    std::vector<float> o((size_t)(nb * c));
    for (int64_t b = 0; b < nb; ++b) std::memcpy(&o[(size_t)(b * c)], &m6[(size_t)(b * 6 * c + i * c)], (size_t)c * 4);
    return o;
}

// The host composition of ModulatedCrossBlock.forward with the chains above.
std::vector<float> host_block(const std::vector<float>& x, const std::vector<float>& m6, const std::vector<float>& w2,
                              const std::vector<float>& b2, const std::vector<int64_t>& offsets, int64_t c) {
    const int64_t rows = (int64_t)x.size() / c, nb = (int64_t)offsets.size() - 1;
    auto mod = [&](const std::vector<float>& v, int i_shift, int i_scale) {
        const auto sh = chunk_rows(m6, nb, c, i_shift), sc = chunk_rows(m6, nb, c, i_scale);
        std::vector<float> o(v.size());
        orc_mod_shift_scale(v.data(), sh.data(), sc.data(), offsets.data(), nb, o.data(), rows, c);
        return o;
    };
    auto h = host_scaled(mod(host_ln(x, c), 0, 1), 0.5f, sp::OP_MUL);
    auto y = host_gated_add(x, h, chunk_rows(m6, nb, c, 2).data(), offsets, c);
    auto h2 = host_scaled(host_ln(y, c, w2.data(), b2.data()), 0.25f, sp::OP_ADD);
    std::vector<float> y2(y.size());
    orc_binop_flat(y.data(), h2.data(), y2.data(), (int64_t)y.size(), sp::OP_ADD);
    auto h3 = host_scaled(mod(host_ln(y2, c), 3, 4), -0.75f, sp::OP_MUL);
    return host_gated_add(y2, h3, chunk_rows(m6, nb, c, 5).data(), offsets, c);
}

void test_modulated_cross_block() {
    const int64_t n = 2, l = 37, c = 1536;
    const auto x = randn(41, n * l * c), mod = randn(42, n * 6 * c, 0.1), par = randn(43, 6 * c, 0.02);
    const auto w2 = randn(44, c, 0.1), b2 = randn(45, c, 0.1);
    std::vector<float> m6((size_t)(n * 6 * c));
    orc_modulation_add(mod.data(), par.data(), m6.data(), n, 6 * c);
    const blk::ModulatedCrossBlock block(c, Tensor::from_host(w2.data(), {c}), Tensor::from_host(b2.data(), {c}),
                                         Tensor::from_host(par.data(), {6 * c}), 1e-6);
    const blk::Chain self_attn = [](const Tensor& h) { return scaled(h, 0.5f, sp::OP_MUL); };
    const blk::Chain cross_attn = [](const Tensor& h) { return scaled(h, 0.25f, sp::OP_ADD); };
    const blk::Chain mlp = [](const Tensor& h) { return scaled(h, -0.75f, sp::OP_MUL); };
    const Tensor modd = Tensor::from_host(mod.data(), {n, 6 * c});
    // dense [N, L, C]: batch b owns rows [b L, (b + 1) L)
    const Tensor out = block.forward(Tensor::from_host(x.data(), {n, l, c}), modd, self_attn, cross_attn, mlp);
    EXPECT((out.shape() == std::vector<int64_t>{n, l, c}));
    expect_close(out.to_host(), host_block(x, m6, w2, b2, {0, l, 2 * l}, c), 1e-5, "ModulatedCrossBlock dense");
    // sparse: three batches, the middle one empty
    const int64_t rows = 90;
    std::vector<int32_t> coords((size_t)rows * 4, 0);
    for (int64_t r = 0; r < rows; ++r) coords[(size_t)r * 4] = r < 50 ? 0 : 2;
    const auto xs = randn(46, rows * c), mods = randn(47, 3 * 6 * c, 0.1);
    std::vector<float> m6s((size_t)(3 * 6 * c));
    orc_modulation_add(mods.data(), par.data(), m6s.data(), 3, 6 * c);
    const sp::SparseTensor st(Tensor::from_host(xs.data(), {rows, c}), IntMatrix::from_host(coords.data(), rows, 4), 3);
    const auto so = block.forward(st, Tensor::from_host(mods.data(), {3, 6 * c}), self_attn, cross_attn, mlp);
    expect_close(so.feats.to_host(), host_block(xs, m6s, w2, b2, {0, 50, 50, rows}, c), 1e-5,
                 "ModulatedCrossBlock sparse");
    expect_error([&] { block.forward(st, modd, self_attn, cross_attn, mlp); }, "batch size mismatch");
    expect_error([&] { block.forward(Tensor::zeros({n, l, c - 8}), modd, self_attn, cross_attn, mlp); },
                 "LayerNorm32: last dim mismatch");
}

void test_cross_block_enqueue() {
    // the resident block over one const buffer; chains return no out bias
    const int64_t rows = 77, c = 1536;
    const auto x = randn(51, rows * c);
    std::vector<Tensor> m;
    std::vector<std::vector<float>> mh;
    for (int i = 0; i < 6; ++i) {
        mh.push_back(randn(52 + i, c, 0.1));
        m.push_back(Tensor::from_host(mh.back().data(), {c}));
    }
    const auto w2 = randn(60, c, 0.1), b2 = randn(61, c, 0.1), bs = randn(62, c, 0.02), bc = randn(63, c, 0.02),
               bm = randn(64, c, 0.02);
    const Tensor bk = blk::pack_block_consts(m, Tensor::from_host(w2.data(), {c}), Tensor::from_host(b2.data(), {c}),
                                             Tensor::from_host(bs.data(), {c}), Tensor::from_host(bc.data(), {c}),
                                             Tensor::from_host(bm.data(), {c}));
    const blk::Chain self_chain = [](const Tensor& h) { return scaled(h, 0.5f, sp::OP_MUL); };
    const blk::Chain cross_chain = [](const Tensor& h) { return h; };   // hands back its input
    const blk::Chain mlp_chain = [](const Tensor& h) { return scaled(h, -0.75f, sp::OP_MUL); };
    Tensor xf = Tensor::from_host(x.data(), {rows, c}), xu = Tensor::from_host(x.data(), {rows, c});
    blk::cross_block_enqueue(xf, bk, self_chain, cross_chain, mlp_chain, true);
    blk::cross_block_enqueue(xu, bk, self_chain, cross_chain, mlp_chain, false);
    const auto got = xf.to_host();
    expect_bits(got, xu.to_host(), "cross_block_enqueue fused == unfused");
    // host: the joins fold the out bias: x += fl(fl(h + bias) * gate)
    const std::vector<int64_t> off{0, rows};
    auto modulate = [&](const std::vector<float>& v, const std::vector<float>& sh, const std::vector<float>& sc) {
        std::vector<float> o(v.size());
        orc_mod_shift_scale(v.data(), sh.data(), sc.data(), off.data(), 1, o.data(), rows, c);
        return o;
    };
    auto add_bias = [&](const std::vector<float>& v, const std::vector<float>& b) {
        std::vector<float> o(v.size());
        orc_add_bias(v.data(), b.data(), o.data(), rows, c);
        return o;
    };
    auto h = host_scaled(modulate(host_ln(x, c), mh[0], mh[1]), 0.5f, sp::OP_MUL);
    auto y = host_gated_add(x, add_bias(h, bs), mh[2].data(), off, c);
    auto h2 = add_bias(host_ln(y, c, w2.data(), b2.data()), bc);
    std::vector<float> y2(y.size());
    orc_binop_flat(y.data(), h2.data(), y2.data(), (int64_t)y.size(), sp::OP_ADD);
    auto h3 = host_scaled(modulate(host_ln(y2, c), mh[3], mh[4]), -0.75f, sp::OP_MUL);
    expect_close(got, host_gated_add(y2, add_bias(h3, bm), mh[5].data(), off, c), 1e-5, "cross_block_enqueue");
    expect_error([&] { blk::pack_block_consts({m[0]}, m[0], m[0]); }, "expected 6 mod chunks");
}

// ---- gpu/linear.mojo, gpu/attention.mojo ---------------------------------------------
namespace gp = t2h::gpu;

// small integers in [-m, m]: exact in f16, their products and sums exact in f32
std::vector<float> small_ints(uint64_t seed, int64_t n, int m) {
    orc_rng r;
    orc_rng_init(&r, seed);
    std::vector<float> v((size_t)n);
    for (auto& x : v) x = (float)((int)(orc_rng_next_u64(&r) % (uint64_t)(2 * m + 1)) - m);
    return v;
}

std::vector<float> host_linear(const std::vector<float>& x, const std::vector<float>& w, int64_t rows, int64_t n,
                               int64_t k) {
    std::vector<float> c((size_t)(rows * n));
    orc_linear(x.data(), w.data(), c.data(), rows, n, k, 4);
    return c;
}

void test_gpu_linear() {
    const int64_t rows = 100, k = 128, n = 256;
    const auto x = small_ints(81, rows * k, 3), w = small_ints(82, n * k, 2), b = small_ints(83, n, 4);
    const Tensor xd = Tensor::from_host(x.data(), {rows, k}, t2h::F16), wd = Tensor::from_host(w.data(), {n, k}, t2h::F16);
    const Tensor bd = Tensor::from_host(b.data(), {n});
    const auto acc = host_linear(x, w, rows, n, k);
    std::vector<float> want(acc.size());
    orc_add_bias(acc.data(), b.data(), want.data(), rows, n);
    expect_bits(gp::linear(xd, wd, bd).to_host(), want, "linear f32 out (integer operands)");
    expect_bits(gp::linear(xd, wd, bd, T2H_ACT_NONE, t2h::F16).to_host(), want, "linear f16 out (integer operands)");
    std::vector<float> act(want.size());
    EXPECT(orc_activation(want.data(), act.data(), (int64_t)want.size(), T2H_ACT_GELU_TANH, 1) == 0);
    expect_close(gp::linear(xd, wd, bd, T2H_ACT_GELU_TANH).to_host(), act, 1e-5, "linear + GELU-tanh");
    // the out-linear with the gated residual join, per-batch gate rows
    const auto res = randn(84, rows * n), gate = randn(85, 2 * n, 0.1);
    const std::vector<int64_t> off{0, 40, rows};
    const sp::VarLenTensor batches(Tensor::zeros({rows, 1}), off);   // device offsets
    const Tensor got = gp::linear_gate_residual(xd, wd, Tensor::from_host(res.data(), {rows, n}), bd,
                                                Tensor::from_host(gate.data(), {2, n}), batches.device_offsets(), 2);
    expect_bits(got.to_host(), host_gated_add(res, want, gate.data(), off, n), "linear_gate_residual");
    expect_error([&] { gp::linear(xd, Tensor::from_host(w.data(), {n, k})); }, "float16 or bfloat16 alike");
}

// The host composition of attn_pack: +bias, RMS q/k, RoPE q/k from coords,
// then pack_q / pack_kv (gpu/attention.mojo:507-662).
struct HostPack {
    std::vector<float> qh, kt, vh;
};
HostPack host_attn_pack(const std::vector<float>& qkv, const std::vector<float>& bias, const std::vector<float>& gq,
                        const std::vector<float>& gk, const std::vector<int32_t>& coords, int64_t rows, int64_t h,
                        int64_t d, int64_t mp, int64_t lp) {
    const int64_t hd = h * d;
    std::vector<float> t(qkv.size());
    orc_add_bias(qkv.data(), bias.data(), t.data(), rows, 3 * hd);
    std::vector<float> freqs((size_t)d / 2);
    const int64_t fd = orc_rope_freqs(d, 3, 1.0, 10000.0, freqs.data());
    std::vector<float> ph((size_t)(rows * d));
    orc_rope_phases_from_coords(coords.data(), rows, 4, 3, d, freqs.data(), fd, ph.data());
    for (int part = 0; part < 2; ++part) {
        std::vector<float> a((size_t)(rows * hd)), r(a.size()), o(a.size());
        for (int64_t i = 0; i < rows; ++i) std::memcpy(&a[(size_t)(i * hd)], &t[(size_t)(i * 3 * hd + part * hd)], (size_t)hd * 4);
        orc_multihead_rmsnorm(a.data(), (part == 0 ? gq : gk).data(), r.data(), rows, h, d, 1);
        orc_rope_rotate(r.data(), ph.data(), o.data(), rows, h, d, 1);
        for (int64_t i = 0; i < rows; ++i) std::memcpy(&t[(size_t)(i * 3 * hd + part * hd)], &o[(size_t)(i * hd)], (size_t)hd * 4);
    }
    HostPack p{std::vector<float>((size_t)(h * mp * d)), std::vector<float>((size_t)(h * d * lp)),
               std::vector<float>((size_t)(h * lp * d))};
    orc_pack_q(t.data(), p.qh.data(), rows, h, d, mp, 3 * hd);
    orc_pack_kv(t.data(), p.kt.data(), p.vh.data(), rows, h, d, lp);
    p.qh = round_f16(p.qh);
    p.kt = round_f16(p.kt);
    p.vh = round_f16(p.vh);
    return p;
}

void test_gpu_attn_pack() {
    const int64_t rows = 70, h = 12, d = 128, hd = h * d, mp = 72, lp = 80, k = 256;
    const auto bias = randn(91, 3 * hd, 0.02), gq = randn(92, hd, 0.02), gk = randn(93, hd, 0.02);
    std::vector<float> gq1(gq), gk1(gk);
    for (auto& v : gq1) v += 1.0f;
    for (auto& v : gk1) v += 1.0f;
    std::vector<int32_t> coords((size_t)rows * 4, 0);
    orc_rng r;
    orc_rng_init(&r, 94);
    for (int64_t i = 0; i < rows; ++i)
        for (int a = 1; a < 4; ++a) coords[(size_t)i * 4 + a] = (int32_t)(orc_rng_next_u64(&r) % 64);
    const IntMatrix cm = IntMatrix::from_host(coords.data(), rows, 4);
    gp::Rope rope;
    rope.freqs = nn::rope_freqs(d);
    rope.coords = &cm;
    const Tensor bd = Tensor::from_host(bias.data(), {3 * hd}), gqd = Tensor::from_host(gq1.data(), {h, d}),
                 gkd = Tensor::from_host(gk1.data(), {h, d});
    auto compare = [&](const gp::AttnOperands& o, const HostPack& want, bool kt, const char* what) {
        expect_close(o.qh.to_host(), want.qh, 2e-3, what);
        expect_close(o.vh.to_host(), want.vh, 2e-3, what);
        if (kt) {
            expect_close(o.k.to_host(), want.kt, 2e-3, what);
        } else {   // [H, lp, D] against the transposed [H, D, lp]
            std::vector<float> krow(want.kt.size());
            for (int64_t z = 0; z < h; ++z)
                for (int64_t e = 0; e < d; ++e)
                    for (int64_t t = 0; t < lp; ++t)
                        krow[(size_t)((z * lp + t) * d + e)] = want.kt[(size_t)((z * d + e) * lp + t)];
            expect_close(o.k.to_host(), krow, 2e-3, what);
        }
    };
    // the epilogue + pack on a qkv GEMM output
    const auto qkv = randn(95, rows * 3 * hd);
    const Tensor qkvd = Tensor::from_host(qkv.data(), {rows, 3 * hd}, t2h::F16);
    const HostPack want = host_attn_pack(round_f16(qkv), bias, gq1, gk1, coords, rows, h, d, mp, lp);
    compare(gp::attn_pack(qkvd, (int32_t)h, bd, gqd, gkd, rope, mp, lp, true), want, true, "attn_pack, k transposed");
    compare(gp::attn_pack(qkvd, (int32_t)h, bd, gqd, gkd, rope, mp, lp, false), want, false, "attn_pack, k row-major");
    // the qkv GEMM with that epilogue and pack in its store
    const auto x = round_f16(randn(96, rows * k, 0.5)), w = round_f16(randn(97, 3 * hd * k, 0.05));
    const HostPack wl = host_attn_pack(host_linear(x, w, rows, 3 * hd, k), bias, gq1, gk1, coords, rows, h, d, mp, lp);
    compare(gp::qkv_linear_pack(Tensor::from_host(x.data(), {rows, k}, t2h::F16),
                                Tensor::from_host(w.data(), {3 * hd, k}, t2h::F16), (int32_t)h, bd, gqd, gkd, rope, mp,
                                lp, true),
            wl, true, "qkv_linear_pack");
    expect_error([&] { gp::attn_pack(qkvd, 7, bd, gqd, gkd); }, "attn_pack: qkv must be [rows, 3 * H * D]");
}

// ---- samplers/flow_euler.mojo --------------------------------------------------------
namespace smp = t2h::samplers;

void test_flow_euler_sampler() {
    // t_schedule: t = 1 -> 1, t = 0 -> 0, rescale_t 1 is linspace(1, 0)
    const auto ts1 = smp::t_schedule(4, 1.0);
    EXPECT(ts1.size() == 5 && ts1[0] == 1.0 && ts1[2] == 0.5 && ts1[4] == 0.0);
    const auto ts3 = smp::t_schedule(4, 3.0);
    EXPECT(ts3[0] == 1.0 && ts3[4] == 0.0 && std::fabs(ts3[2] - 0.75) < 1e-15);   // 3 * 0.5 / (1 + 2 * 0.5)
    // model: pos = fl(x * 0.75), neg = fl(fl(x * 0.25) + 0.5): bit-exact on both sides
    const smp::Model model = [](const Tensor& x, double, bool neg) {
        return neg ? scaled(scaled(x, 0.25f, sp::OP_MUL), 0.5f, sp::OP_ADD) : scaled(x, 0.75f, sp::OP_MUL);
    };
    auto host_model = [](const std::vector<float>& x, bool neg) {
        return neg ? host_scaled(host_scaled(x, 0.25f, sp::OP_MUL), 0.5f, sp::OP_ADD) : host_scaled(x, 0.75f, sp::OP_MUL);
    };
    const int64_t rows = 64, rs = 32;
    const double sigma_min = 1e-5;
    const auto noise = randn(71, rows * rs);
    struct Case {
        const char* name;
        int mode;
        double g, lo, hi, gr;
        std::vector<int64_t> seg;
    };
    const std::vector<Case> cases = {
        {"sample", smp::GUIDANCE_NONE, 1.0, 0.0, 1.0, 0.0, {}},
        {"sample_cfg", smp::GUIDANCE_CFG, 3.0, 0.0, 1.0, 0.0, {}},
        {"sample_cfg rescale", smp::GUIDANCE_CFG, 3.0, 0.0, 1.0, 0.7, {}},
        {"sample_cfg strength 0", smp::GUIDANCE_CFG, 0.0, 0.0, 1.0, 0.7, {}},
        {"sample_cfg_interval rescale", smp::GUIDANCE_CFG_INTERVAL, 3.0, 0.3, 0.8, 0.7, {}},
        {"sample_cfg varlen rescale", smp::GUIDANCE_CFG, 3.0, 0.0, 1.0, 0.7, {0, 20, 64}},
    };
    const int steps = 5;
    const auto ts = smp::t_schedule(steps, 3.0);
    for (const Case& k : cases) {
        smp::FlowEulerSampler sampler(sigma_min);
        const Tensor nd = Tensor::from_host(noise.data(), {rows, rs});
        smp::SampleResult res;
        if (k.mode == smp::GUIDANCE_NONE) res = sampler.sample(model, nd, steps, 3.0);
        else if (k.mode == smp::GUIDANCE_CFG) res = sampler.sample_cfg(model, nd, steps, 3.0, k.g, k.gr, k.seg);
        else res = sampler.sample_cfg_interval(model, nd, steps, 3.0, k.g, k.lo, k.hi, k.gr, k.seg);
        EXPECT((int)res.pred_x_t.size() == steps && (int)res.pred_x_0.size() == steps);
        // host: _inference's branches, then the Euler step (flow_euler.mojo:151-214)
        std::vector<float> x = noise;
        const bool rescaled = k.gr > 0.0;
        const double tol = rescaled ? 1e-4 : 0.0;
        for (int i = 0; i < steps; ++i) {
            const double t = ts[(size_t)i], tp = ts[(size_t)i + 1];
            bool use_cfg = k.mode == smp::GUIDANCE_CFG;
            if (k.mode == smp::GUIDANCE_CFG_INTERVAL) use_cfg = k.lo <= t && t <= k.hi;
            std::vector<float> v;
            if (!use_cfg || k.g == 1.0) {
                v = host_model(x, false);
            } else if (k.g == 0.0) {
                v = host_model(x, true);
            } else {
                const auto pos = host_model(x, false), neg = host_model(x, true);
                v.resize(x.size());
                orc_flow_cfg(pos.data(), neg.data(), v.data(), (int64_t)x.size(), k.g);
                if (rescaled) {
                    std::vector<float> r(x.size());
                    orc_flow_rescale(x.data(), v.data(), pos.data(), r.data(), rows, rs, t, sigma_min, k.gr,
                                     k.seg.empty() ? nullptr : k.seg.data(), (int64_t)k.seg.size());
                    v = r;
                }
            }
            std::vector<float> x0(x.size()), xn(x.size());
            orc_flow_v_to_xstart(x.data(), v.data(), x0.data(), (int64_t)x.size(), t, sigma_min);
            orc_flow_step(x.data(), v.data(), xn.data(), (int64_t)x.size(), t, tp);
            x = xn;
            if (tol == 0.0) {
                expect_bits(res.pred_x_0[(size_t)i].to_host(), x0, k.name);
                expect_bits(res.pred_x_t[(size_t)i].to_host(), x, k.name);
            } else {
                expect_close(res.pred_x_0[(size_t)i].to_host(), x0, tol, k.name);
                expect_close(res.pred_x_t[(size_t)i].to_host(), x, tol, k.name);
            }
        }
        EXPECT(std::memcmp(res.samples.to_host().data(), res.pred_x_t.back().to_host().data(), x.size() * 4) == 0);
    }
}

// ---- host side of the header (no GPU) ------------------------------------------------
bool same_value(float a, float b) {
    if (std::isnan(a) || std::isnan(b)) return std::isnan(a) && std::isnan(b);
    return std::memcmp(&a, &b, 4) == 0;
}

void test_host_f16_conversion() {
    // every f16 pattern decodes as the oracle's, and encodes back to itself
    for (uint32_t h = 0; h < 65536; ++h) {
        const float f = t2h::detail::f16_to_f32((uint16_t)h);
        EXPECT(same_value(f, orc_f16_to_f32((uint16_t)h)));
        if (!std::isnan(f)) EXPECT(t2h::detail::f32_to_f16(f) == h);
    }
    // f32 -> f16 on random bit patterns and the rounding boundaries
    orc_rng r;
    orc_rng_init(&r, 99);
    std::vector<float> xs = {0.0f, -0.0f, 65504.0f, 65519.99f, 65520.0f, 65536.0f, 1e-8f, 2.98e-8f, 2.9802322e-8f,
                             5.9604645e-8f, 6.1035156e-5f, 6.097555e-5f, INFINITY, -INFINITY, NAN};
    for (int i = 0; i < 1 << 20; ++i) {
        const uint32_t u = (uint32_t)orc_rng_next_u64(&r);
        float f;
        std::memcpy(&f, &u, 4);
        xs.push_back(f);
        xs.push_back(std::ldexp((float)(u >> 8), -40 + (int)(u & 63)));   // the f16 range, finely
    }
    for (float f : xs) {
        const uint16_t got = t2h::detail::f32_to_f16(f), want = orc_f32_to_f16(f);
        if (std::isnan(f)) {
            EXPECT((got & 0x7C00u) == 0x7C00u && (got & 0x3FFu) != 0);
        } else if (got != want) {
            throw Failure{"f32_to_f16 differs at " + std::to_string(f)};
        }
    }
    std::vector<float> rb(xs.size());
    orc_round_bf16(xs.data(), rb.data(), (int64_t)xs.size());
    for (size_t i = 0; i < xs.size(); ++i)
        EXPECT(same_value(t2h::detail::bf16_to_f32(t2h::detail::f32_to_bf16(xs[i])), rb[i]));
    std::printf("    f16 / bf16 storage conversions equal the oracle's (%zu values)\n", xs.size());
}

// The argument checks that come before any device call, with the reference's
// messages (modules/nn.mojo:588-647; modules/rope.mojo:24-37;
// sparse/basic.mojo:89-104) and the library's own for a host-side failure.
void test_host_errors() {
    expect_error([] { nn::activation(Tensor(), 7); }, "unknown activation");
    expect_error([] { nn::RotaryPositionEmbedder(63); }, "RotaryPositionEmbedder: head_dim must be even");
    expect_error([] { sp::SparseRotaryPositionEmbedder(63); }, "SparseRotaryPositionEmbedder: head_dim must be even");
    expect_error([] { nn::rope_freqs(7); }, "head_dim");
    expect_error([] { sp::VarLenTensor(Tensor(), {0, 3, 2, 5}); }, "VarLenTensor: invalid offsets");
    expect_error([] { Tensor::from_values({2, 2}, {1, 2, 3}); }, "Tensor.from_values: size mismatch");
    const std::vector<float> f = nn::rope_freqs(128);
    std::vector<float> want(64);
    EXPECT(orc_rope_freqs(128, 3, 1.0, 10000.0, want.data()) == (int64_t)f.size());
    EXPECT(std::memcmp(f.data(), want.data(), f.size() * 4) == 0);
    std::printf("    argument errors raise t2h::Error with the reference's messages\n");
}

void test_abi_errors_propagate() {
    // a status from libt2h arrives as t2h::Error with the library's message
    expect_error([] { nn::rope_freqs(7); }, "head_dim");
    expect_error([] { nn::TimestepEmbedder(4096).timestep_embedding(Tensor::zeros({2})); }, "timestep");
}

}  // namespace

int main(int argc, char** argv) {
    const std::vector<std::pair<const char*, std::function<void()>>> tests = {
        {"varlen_shape_and_layout", test_varlen_shape_and_layout},
        {"varlen_elemwise", test_varlen_elemwise},
        {"sparse_layout_from_coords", test_sparse_layout_from_coords},
        {"sparse_contiguity_enforced", test_sparse_contiguity_enforced},
        {"sparse_elemwise_batch", test_sparse_elemwise_batch},
        {"layernorm32", test_layernorm32},
        {"modulate_and_gate", test_modulate_and_gate},
        {"mod_shift_scale_sparse", test_mod_shift_scale_sparse},
        {"activation", test_activation},
        {"multihead_rmsnorm_and_rope", test_multihead_rmsnorm_and_rope},
        {"sparse_rope_embed", test_sparse_rope_embed},
        {"timestep_embedder", test_timestep_embedder},
        {"modulation_chunks", test_modulation_chunks},
        {"modulated_cross_block", test_modulated_cross_block},
        {"cross_block_enqueue", test_cross_block_enqueue},
        {"flow_euler_sampler", test_flow_euler_sampler},
        {"gpu_linear", test_gpu_linear},
        {"gpu_attn_pack", test_gpu_attn_pack},
        {"abi_errors_propagate", test_abi_errors_propagate},
    };
    if (argc > 1 && std::strcmp(argv[1], "--host") == 0) {   // the checks that need no GPU
        const std::vector<std::pair<const char*, std::function<void()>>> host_tests = {
            {"host_f16_conversion", test_host_f16_conversion},
            {"host_errors", test_host_errors},
        };
        int failed = 0;
        for (const auto& t : host_tests) {
            std::printf("test %s\n", t.first);
            try {
                t.second();
                std::printf("ok %s\n", t.first);
            } catch (const Failure& f) {
                ++failed;
                std::printf("FAIL %s: %s\n", t.first, f.what.c_str());
            } catch (const std::exception& e) {
                ++failed;
                std::printf("FAIL %s: unexpected exception: %s\n", t.first, e.what());
            }
        }
        return failed == 0 ? 0 : 1;
    }
    const char* filter = argc > 1 ? argv[1] : nullptr;
    if (t2h_device_init(0) != T2H_OK) {
        std::printf("t2h_device_init: %s\n", t2h_last_error());
        return 2;
    }
    int failed = 0, ran = 0;
    for (const auto& t : tests) {
        if (filter != nullptr && std::strstr(t.first, filter) == nullptr) continue;
        std::printf("test %s\n", t.first);
        std::fflush(stdout);
        ++ran;
        try {
            t.second();
            std::printf("ok %s\n", t.first);
        } catch (const Failure& f) {
            ++failed;
            std::printf("FAIL %s: %s\n", t.first, f.what.c_str());
        } catch (const std::exception& e) {
            ++failed;
            std::printf("FAIL %s: unexpected exception: %s\n", t.first, e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%d of %d passed\n", ran - failed, ran);
    return failed == 0 && ran > 0 ? 0 : 1;
}
