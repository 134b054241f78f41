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

typedef int (*Launch)(const void*, void*, const float*, int64_t, hipStream_t);
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
