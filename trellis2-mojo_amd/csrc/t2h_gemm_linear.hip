// The weight GEMM's linear and gated-residual kernels and their launchers:
// t2h_linear (out = act(acc + bias)) and t2h_linear_gate_residual (out = res +
// fl(fl(acc + bias) * gate[b(t)])), on the 8-wave, register-staged layout of
// the GEMM core (tiling and pipeline: t2h_gemm_core.h).
//
// Reference: GpuLinear.enqueue_gemm (gpu/linear.mojo:535-560), the MLP's
// lin0 + gelu_tanh_bias (gpu/linear.mojo:662-684, 776-809), the out-linears
// + gate_add_bias_rows (gpu/block.mojo:86-110, 317-397).
#define T2H_GEMM_WAVES 8
#include "t2h_gemm_core.h"

namespace t2h {
namespace {

// ---- linear: out = act(acc + bias) ------------------------------------------
// The lane holds token wt*kWT + tj*32 + fr of each token tile and features
// wf*kWF + fi*32 + 8q + 4h + 0..3. bias + activation are applied in f32 on
// the accumulators (one rounding to the output type). 16-bit outputs are
// staged in LDS as 256 token rows of 512 bytes (16-byte chunk c of row r at
// c ^ (r % 32): conflict-free both ways) and leave as whole rows, 16
// contiguous bytes per lane; f32 outputs go out directly.
template <typename T, typename O, int ACT>
__global__ __launch_bounds__(kGemmThreads, T2H_GEMM_OCC) void gemm_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];
    TileOf tile;
    if (!tile.init(a)) return;
    const int64_t t0 = tile.t0, n0 = tile.n0;
    f32x16 acc[kFI][kTJ];
    zero_acc(acc);
    gemm_mainloop<T>(a, t0, n0, lds, acc);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wf = wave & 1, wt = wave >> 1;
    const int fr = lane & 31, h = lane >> 5;
    O* __restrict__ out = static_cast<O*>(a.out);
    auto bias4 = [&](int fi, int q, float* bq) {
        if (a.bias != nullptr) {
            load_params<4>(a.bias + n0 + wf * kWF + fi * 32 + q * 8 + h * 4, bq);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) bq[i] = 0.0f;
        }
    };
    if constexpr (sizeof(O) == 2) {
        static_assert(kBT * kBF * 2 <= kStages * kStageBytes, "C tile fits the stage buffers");
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
            float bv[4][4];
#pragma unroll
            for (int q = 0; q < 4; ++q) bias4(fi, q, bv[q]);
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int r = wt * kWT + tj * 32 + fr;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int c = (wf * kWF + fi * 32 + q * 8) / 8;
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = epi_f<ACT>(acc[fi][tj][q * 4 + i], bv[q][i]);
                    u32x2 w;
                    w.x = Word<O>::pack(v);
                    w.y = Word<O>::pack(v + 2);
                    *reinterpret_cast<u32x2*>(lds + r * (kBF * 2) + ((c ^ (r & 31)) * 16) + h * 8) = w;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        constexpr int kRowsPerWave = kBT / kWaves;
#pragma unroll 4
        for (int it = 0; it < kRowsPerWave / 2; ++it) {
            const int r = wave * kRowsPerWave + it * 2 + h;
            const int c = fr;
            const int64_t t = t0 + r;
            const u32x4 w = *reinterpret_cast<const u32x4*>(lds + r * (kBF * 2) + ((c ^ (r & 31)) * 16));
            if (t < a.rows) out_store16(out + t * a.ldo + n0 + c * 8, w);
        }
    } else {
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
            float bv[4][4];
#pragma unroll
            for (int q = 0; q < 4; ++q) bias4(fi, q, bv[q]);
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int64_t t = t0 + wt * kWT + tj * 32 + fr;
                if (t >= a.rows) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t n = n0 + wf * kWF + fi * 32 + q * 8 + h * 4;
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = epi_f<ACT>(acc[fi][tj][q * 4 + i], bv[q][i]);
                    store_elems<O, 4, T2H_GEMM_NTS>(out + t * a.ldo + n, v);
                }
            }
        }
    }
}

// ---- linear + gated residual: out = res + fl(fl(acc + bias) * gate[b(t)]) ----
// The residual join of the block (x += (h + bias) * gate, or x += h + bias)
// in the store of the GEMM that makes h, so h never reaches memory; the
// rounding sequence is the gated-residual kernel's, with h = the f32 sums.
// 16-bit outputs: the residual tile is copied into the freed LDS stages with
// direct-to-LDS loads (each lane fetches the chunk that the staging swizzle
// puts at its slot; the half that lands in the stage buffer the last k step
// leaves free is requested before that step's MFMAs), each lane updates its
// values there in place, and whole rows leave as 16-byte stores. f32 outputs
// read and write the residual directly. out may alias res (every element is
// read before it is written, by the same thread).
template <typename T, typename O>
__global__ __launch_bounds__(kGemmThreads, T2H_GEMM_OCC) void gemm_res_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];
    TileOf tile;
    if (!tile.init(a)) return;
    const int64_t t0 = tile.t0, n0 = tile.n0;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wf = wave & 1, wt = wave >> 1;
    const int fr = lane & 31, h = lane >> 5;
    const BatchMap bm{a.batch.offsets, a.batch.rows_per_batch, a.batch.nbatch};
    const O* __restrict__ res = static_cast<const O*>(a.res);
    O* __restrict__ out = static_cast<O*>(a.out);
    const int64_t last = a.rows - 1;
    // gate row of the tile when all its rows share one batch (block-uniform),
    // else -1: each token looks up its own
    f32x16 acc[kFI][kTJ];
    zero_acc(acc);
    gemm_mainloop<T, sizeof(O) == 2>(a, t0, n0, lds, acc);
    int64_t tile_b = 0;
    if (a.gate != nullptr) {
        const int64_t tl = t0 + kBT - 1 < last ? t0 + kBT - 1 : last;
        const int32_t b0 = bm.batch_of(t0 < last ? t0 : last);
        tile_b = bm.batch_of(tl) == b0 ? b0 : -1;
    }
    // bias and gate of feature group fi (4 runs of 4 features per lane)
    auto params = [&](int fi, float (&bv)[4][4], float (&gv)[4][4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int64_t n = n0 + wf * kWF + fi * 32 + q * 8 + h * 4;
            if (a.bias != nullptr) load_params<4>(a.bias + n, bv[q]);
            if (a.gate != nullptr && tile_b >= 0) load_params<4>(a.gate + tile_b * a.gate_stride + n, gv[q]);
        }
    };
    // u = res + fl(fl(acc + bias) * gate) for token tile tj, group (fi, q)
    auto join4 = [&](int fi, int tj, int q, const float* bq, const float* gq, const float* rv, float* u) {
        float g[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) g[i] = gq[i];
        if (a.gate != nullptr && tile_b < 0) {
            const int64_t t = t0 + wt * kWT + tj * 32 + fr;
            load_params<4>(a.gate + bm.batch_of(t < last ? t : last) * a.gate_stride + n0 + wf * kWF + fi * 32 +
                               q * 8 + h * 4, g);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = a.bias != nullptr ? add_rn(acc[fi][tj][q * 4 + i], bq[i]) : acc[fi][tj][q * 4 + i];
            if (a.gate != nullptr) v = mul_rn(v, g[i]);
            u[i] = add_rn(rv[i], v);
        }
    };
    if constexpr (sizeof(O) == 2) {
        static_assert(kBT * kBF * 2 <= kStages * kStageBytes, "C tile fits the stage buffers");
        constexpr int kRowsPerWave = kBT / kWaves;
        // residual rows -> LDS: the last stage left rows [128 * (ksteps % 2),
        // +128) loading; now the other half
        res_rows(a, t0, n0, lds, (1 - (a.k / kBK) % 2) * 128, wave, lane);
        wait_vm<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
            float bv[4][4], gv[4][4];
            params(fi, bv, gv);
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int r = wt * kWT + tj * 32 + fr;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int c = (wf * kWF + fi * 32 + q * 8) / 8;
                    u32x2* p = reinterpret_cast<u32x2*>(lds + r * (kBF * 2) + ((c ^ (r & 31)) * 16) + h * 8);
                    const u32x2 w0 = *p;
                    float rv[4], u[4];
                    Word<O>::unpack(w0.x, rv);
                    Word<O>::unpack(w0.y, rv + 2);
                    join4(fi, tj, q, bv[q], gv[q], rv, u);
                    u32x2 w;
                    w.x = Word<O>::pack(u);
                    w.y = Word<O>::pack(u + 2);
                    *p = w;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
#pragma unroll 4
        for (int it = 0; it < kRowsPerWave / 2; ++it) {
            const int r = wave * kRowsPerWave + it * 2 + h;
            const int c = fr;
            const int64_t t = t0 + r;
            const u32x4 w = *reinterpret_cast<const u32x4*>(lds + r * (kBF * 2) + ((c ^ (r & 31)) * 16));
            if (t < a.rows) out_store16(out + t * a.ldo + n0 + c * 8, w);
        }
    } else {
        // per feature group: its residual values and parameters are all
        // loaded before its first store (loads and stores share vmcnt on
        // gfx9: a load consumed while a store is pending waits for the store)
#pragma unroll
        for (int fi = 0; fi < kFI; ++fi) {
            float bv[4][4], gv[4][4];
            params(fi, bv, gv);
            float rv[kTJ][4][4];
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int64_t t = t0 + wt * kWT + tj * 32 + fr;
                const int64_t tc = t < a.rows ? t : last;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    load_elems<O, 4>(res + tc * a.ldo + n0 + wf * kWF + fi * 32 + q * 8 + h * 4, rv[tj][q]);
            }
#pragma unroll
            for (int tj = 0; tj < kTJ; ++tj) {
                const int64_t t = t0 + wt * kWT + tj * 32 + fr;
                if (t >= a.rows) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float u[4];
                    join4(fi, tj, q, bv[q], gv[q], rv[tj][q], u);
                    store_elems<O, 4, T2H_GEMM_NTS>(out + t * a.ldo + n0 + wf * kWF + fi * 32 + q * 8 + h * 4, u);
                }
            }
        }
    }
}

template <typename T, typename O>
hipError_t gemm_act(const GemmArgs& a, hipStream_t s) {
    const dim3 g = grid_1d(a.nblocks), blk(kGemmThreads);
    switch (a.act) {
        case T2H_ACT_RELU: hipLaunchKernelGGL((gemm_kernel<T, O, T2H_ACT_RELU>), g, blk, 0, s, a); break;
        case T2H_ACT_SILU: hipLaunchKernelGGL((gemm_kernel<T, O, T2H_ACT_SILU>), g, blk, 0, s, a); break;
        case T2H_ACT_GELU: hipLaunchKernelGGL((gemm_kernel<T, O, T2H_ACT_GELU>), g, blk, 0, s, a); break;
        case T2H_ACT_GELU_TANH: hipLaunchKernelGGL((gemm_kernel<T, O, T2H_ACT_GELU_TANH>), g, blk, 0, s, a); break;
        default: hipLaunchKernelGGL((gemm_kernel<T, O, -1>), g, blk, 0, s, a); break;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t gemm_typed(const GemmArgs& a, hipStream_t s) {
    if (a.out_dtype == T2H_F32) return gemm_act<T, float>(a, s);
    return gemm_act<T, T>(a, s);
}

template <typename T>
hipError_t gemm_res_typed(const GemmArgs& a, hipStream_t s) {
    const dim3 g = grid_1d(a.nblocks), blk(kGemmThreads);
    if (a.out_dtype == T2H_F32) hipLaunchKernelGGL((gemm_res_kernel<T, float>), g, blk, 0, s, a);
    else hipLaunchKernelGGL((gemm_res_kernel<T, T>), g, blk, 0, s, a);
    return hipGetLastError();
}

}  // namespace

int32_t gemm_feature_tile() { return kBF; }
int32_t gemm_k_step() { return kBK; }

hipError_t launch_gemm(GemmArgs a, hipStream_t s) {
    a.ftiles = a.n / kBF;
    a.nblocks = ((a.rows + kBT - 1) / kBT) * a.ftiles;
    a.tgroup = tile_group(a.k);
    if (a.nblocks == 0) return hipSuccess;
    if (a.dtype == T2H_F16) return gemm_typed<_Float16>(a, s);
    return gemm_typed<__bf16>(a, s);
}

hipError_t launch_gemm_residual(GemmArgs a, hipStream_t s) {
    a.ftiles = a.n / kBF;
    a.nblocks = ((a.rows + kBT - 1) / kBT) * a.ftiles;
    a.tgroup = tile_group(a.k);
    if (a.nblocks == 0) return hipSuccess;
    if (a.dtype == T2H_F16) return gemm_res_typed<_Float16>(a, s);
    return gemm_res_typed<__bf16>(a, s);
}

}  // namespace t2h
