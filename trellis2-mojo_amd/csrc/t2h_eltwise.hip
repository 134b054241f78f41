// Elementwise token-row ops: activation(+bias), gated residual, modulate,
// batch-broadcast binop, sinusoidal timestep embedding, coords -> batch
// offsets, share_mod modulation add.
//
// Row-tiled layout: a block covers RPT consecutive rows and block_threads * V
// columns (V = 16 B of storage per thread; one whole row when it fits). Per-column parameters (bias)
// are loaded once per thread; per-batch parameter rows (gate, shift/scale,
// `other`) are reloaded only when the tile's row crosses a batch boundary
// (the batch of a row is block-uniform). All RPT rows are loaded before any
// is computed so each thread keeps RPT x 16 B per stream in flight. No
// integer division per element: the column comes from the thread index.
//
// Reference: modules/nn.mojo:588-647 (activation), 660-689 (modulate);
// modules/transformer/modulated.mojo:22-33 (_gate); sparse/tensor.mojo:
// 193-219 (_binop_flat/_binop_rows); sparse/transformer/modulated.mojo:60-65;
// gpu/block.mojo:86-110 (gate_add_bias_rows); gpu/linear.mojo:662-684
// (gelu_tanh_bias); models/sparse_structure_flow.mojo:60-76 (timestep);
// sparse/basic.mojo:321-339 (_cal_offsets).
#include "t2h_device.h"
#include "t2h_internal.h"
#include "t2h_act.h"

namespace t2h {
namespace {

constexpr int kBlock = 256;
#ifndef T2H_ELT_RPT
#define T2H_ELT_RPT 4
#endif
constexpr int kRpt = T2H_ELT_RPT;  // rows per thread

// Vector (V = 16 B) or scalar (V = 1) access to V elements of a row.
template <typename T, int V>
__device__ __forceinline__ void ld(const T* p, float* f) {
    if constexpr (V == 1) f[0] = ld1(p);
    else load_elems<T, V, true>(p, f);
}
template <typename T, int V>
__device__ __forceinline__ void st(T* p, const float* f) {
    if constexpr (V == 1) st1(p, f[0]);
    else store_elems<T, V, true>(p, f);
}
template <int V>
__device__ __forceinline__ void ldp(const float* p, float* f) {
    if constexpr (V == 1) f[0] = *p;
    else load_params<V>(p, f);
}

struct Tile {
    int64_t col0;
    int64_t r0;
    int nrows;
    // Row k of the tile for loads, clamped to the tile's last row: every load
    // is unconditional (so all kRpt loads are in flight together) and only the
    // stores check k < nrows.
    __device__ __forceinline__ int64_t row(int k) const { return r0 + (k < nrows ? k : nrows - 1); }
};

// Tile of this block, 1-D grid. When a row is a whole number of waves of
// 16-byte vectors (cols / V = block_threads <= 1024), a block is exactly one row
// wide and covers kRpt full rows: every thread is busy and the block streams
// one contiguous span. Otherwise blocks are kBlock * V columns wide and
// consecutive blocks walk the column tiles of a row tile first, so blocks
// that run together still stream contiguous rows. The column-tile count comes
// from the host: no 64-bit division per wave, none at all for row-wide blocks.
template <int V>
__device__ __forceinline__ bool tile_of(const EltArgs& a, Tile& t) {
    const int64_t b = front_of(block_linear(), a.fper);
    int64_t rt, cb;
    if (a.col_tiles == 1) {
        rt = b;
        cb = 0;
    } else {
        rt = b / a.col_tiles;
        cb = b - rt * a.col_tiles;
    }
    t.col0 = (cb * a.block_threads + threadIdx.x) * V;
    t.r0 = rt * kRpt;
    if (t.r0 >= a.rows) return false;   // past the last row tile of a 2-D grid
    const int64_t left = a.rows - t.r0;
    t.nrows = left < kRpt ? (int)left : kRpt;
    return t.col0 < a.cols;
}

// ---- activation(x + bias) ----------------------------------------------------

// Stores the tile's rows after all of them are computed. Loads and stores
// share vmcnt on gfx9, so a load consumed while a store is pending waits for
// vmcnt(0), i.e. for the store to complete; the per-batch parameter loads of
// the row loop therefore all come before the first store.
template <typename T, int V>
__device__ __forceinline__ void store_rows(T* __restrict__ o, int64_t cols, const Tile& t, const float (&v)[kRpt][V]) {
#pragma unroll
    for (int k = 0; k < kRpt; ++k) {
        if (k >= t.nrows) break;
        st<T, V>(o + (t.r0 + k) * cols + t.col0, v[k]);
    }
}

template <typename T, int V, int KIND, bool BIAS>
__global__ __launch_bounds__(1024) void act_kernel(EltArgs a) {
    Tile t;
    if (!tile_of<V>(a, t)) return;
    const T* __restrict__ x = static_cast<const T*>(a.x);
    T* __restrict__ o = static_cast<T*>(a.out);
    float bias[V];
    if (BIAS) ldp<V>(a.bias + t.col0, bias);
    // Row loads stay conditional here: one load in flight per thread and row
    // streams faster for this kernel than issuing all kRpt loads up front,
    // also when the rows are kept packed until their math (measured on
    // MI355X: 813 vs 842 us on config 5).
    float v[kRpt][V];
#pragma unroll
    for (int k = 0; k < kRpt; ++k)
        if (k < t.nrows) ld<T, V>(x + (t.r0 + k) * a.cols + t.col0, v[k]);
#pragma unroll
    for (int k = 0; k < kRpt; ++k) {
        if (k >= t.nrows) break;
#pragma unroll
        for (int i = 0; i < V; ++i) v[k][i] = act_f<KIND>(BIAS ? bias_add(v[k][i], bias[i]) : v[k][i]);
        st<T, V>(o + (t.r0 + k) * a.cols + t.col0, v[k]);
    }
}

// Slab layout, one vector per thread: a wave covers 64 vectors (64 * V
// columns, 1 KB) of one row, a block covers that column slab for kSlabRows
// consecutive rows, and consecutive blocks walk the slabs of a row tile
// (2-D grid: x = slab, y = row tile, dispatched x first; no index division).
// Every thread moves exactly one 16-byte vector in and one out. The slab's
// bias is read from global memory once per block (16 B for each thread of
// the first V / 4 waves) into LDS, behind an LDS-only barrier that leaves the
// row loads in flight. Measured on MI355X (config-5 GELU, f16
// [201436, 6144]): one row per thread streams at ~84 % of HBM peak where the
// several rows per thread that per-thread bias loads need to amortise stay
// at ~76 %. Each wave lives for one load and one store, so its start-up
// counts: the kernel takes a small argument block (one scalar load round)
// and writes the bias to LDS in thread order (no bank conflicts on the
// 16-byte stores).
constexpr int kSlabRows = 4;
constexpr int kSlabThreads = 64 * kSlabRows;

struct SlabArgs {
    const void* x;
    void* out;
    const float* bias;
    int64_t rows;
    int32_t cols;
};

template <typename T, int V, int KIND, bool BIAS>
__global__ __launch_bounds__(kSlabThreads) void act_slab_kernel(SlabArgs a) {
    constexpr int Q = V / 4;   // float4 pieces of a lane's bias
    __shared__ float4 bl[BIAS ? 64 * Q : 1];   // the slab's bias in column order
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c0 = (int)blockIdx.x * (64 * V);   // < cols <= 2^31 - 1
    const int64_t r = (int64_t)blockIdx.y * kSlabRows + wave;
    const int col = c0 + lane * V;
    const bool live = r < a.rows && col < a.cols;
    float4 bq;
    if (BIAS && wave < Q) {
        // slab floats [4 * tid, 4 * tid + 4), clamped to the row (cols % 4 == 0)
        const int f = 4 * tid < a.cols - c0 ? c0 + 4 * tid : a.cols - 4;
        bq = *reinterpret_cast<const float4*>(a.bias + f);
    }
    // The row load is unconditional (indices clamped), so no lane's load sits
    // behind a branch that would make the bias wait for it.
    float v[V];
    {
        const int64_t rl = r < a.rows ? r : a.rows - 1;
        const int cl = col < a.cols ? col : a.cols - V;
        ld<T, V>(static_cast<const T*>(a.x) + rl * a.cols + cl, v);
    }
    float bias[V];
    if constexpr (BIAS) {
        if (wave < Q) bl[tid] = bq;
        lds_barrier();
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const float4 w = bl[lane * Q + q];
            bias[4 * q] = w.x; bias[4 * q + 1] = w.y; bias[4 * q + 2] = w.z; bias[4 * q + 3] = w.w;
        }
    }
    if (!live) return;
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = act_f<KIND>(BIAS ? bias_add(v[i], bias[i]) : v[i]);
    st<T, V>(static_cast<T*>(a.out) + r * a.cols + col, v);
}

// ---- out = x + fl(fl(h + bias) * gate[b]) ------------------------------------
template <typename T, int V>
__global__ __launch_bounds__(1024) void gate_res_kernel(EltArgs a) {
    Tile t;
    if (!tile_of<V>(a, t)) return;
    const T* __restrict__ x = static_cast<const T*>(a.x);
    const T* __restrict__ h = static_cast<const T*>(a.h);
    T* __restrict__ o = static_cast<T*>(a.out);
    const BatchMap bm{a.batch.offsets, a.batch.rows_per_batch, a.batch.nbatch};
    float bias[V], g[V];
    if (a.bias) ldp<V>(a.bias + t.col0, bias);
    int32_t cur = -1;
    const T* __restrict__ xs = x != nullptr ? x : h;   // without x: a second (ignored) read of h
    float hv[kRpt][V], xv[kRpt][V];
#pragma unroll
    for (int k = 0; k < kRpt; ++k) {
        const int64_t off = t.row(k) * a.cols + t.col0;
        ld<T, V>(h + off, hv[k]);
        // large launches: the residual's first row of the tile with the
        // default cache policy (a buffer load: not merged with its
        // non-temporal twins)
        if (V > 1 && k == 0 && a.cached)
            load_elems_cached<T, V>(xs + t.row(k) * a.cols, t.col0, a.cols, xv[k]);
        else
            ld<T, V>(xs + off, xv[k]);
    }
#pragma unroll
    for (int k = 0; k < kRpt; ++k) {
        if (k >= t.nrows) break;
        const int64_t r = t.r0 + k;
        if (a.gate) {
            const int32_t b = bm.batch_of(r);
            if (b != cur) { ldp<V>(a.gate + b * a.p_stride + t.col0, g); cur = b; }
        }
#pragma unroll
        for (int i = 0; i < V; ++i) {
            float u = a.bias ? add_rn(hv[k][i], bias[i]) : hv[k][i];
            if (a.gate) u = mul_rn(u, g[i]);
            hv[k][i] = x ? add_rn(xv[k][i], u) : u;
        }
    }
    store_rows<T, V>(o, a.cols, t, hv);
}


// ---- out = fl(fl(x * fl(1 + scale[b])) + shift[b]) ---------------------------
template <typename T, int V>
__global__ __launch_bounds__(1024) void modulate_kernel(EltArgs a) {
    Tile t;
    if (!tile_of<V>(a, t)) return;
    const T* __restrict__ x = static_cast<const T*>(a.x);
    T* __restrict__ o = static_cast<T*>(a.out);
    const BatchMap bm{a.batch.offsets, a.batch.rows_per_batch, a.batch.nbatch};
    float sc1[V], sh[V];
    int32_t cur = -1;
    float v[kRpt][V];
#pragma unroll
    for (int k = 0; k < kRpt; ++k) ld<T, V>(x + t.row(k) * a.cols + t.col0, v[k]);
#pragma unroll
    for (int k = 0; k < kRpt; ++k) {
        if (k >= t.nrows) break;
        const int64_t r = t.r0 + k;
        const int32_t b = bm.batch_of(r);
        if (b != cur) {
            ldp<V>(a.gate + b * a.p_stride + t.col0, sc1);
            ldp<V>(a.shift + b * a.p_stride + t.col0, sh);
#pragma unroll
            for (int i = 0; i < V; ++i) sc1[i] = add_rn(1.0f, sc1[i]);
            cur = b;
        }
#pragma unroll
        for (int i = 0; i < V; ++i) v[k][i] = add_rn(mul_rn(v[k][i], sc1[i]), sh[i]);
    }
    store_rows<T, V>(o, a.cols, t, v);
}

// ---- out = x OP other[b] (other row of cols, or one scalar per batch) ---------
__device__ __forceinline__ float apply_op(float x, float y, int op) {
    switch (op) {
        case T2H_OP_ADD: return add_rn(x, y);
        case T2H_OP_SUB: return sub_rn(x, y);
        case T2H_OP_MUL: return mul_rn(x, y);
        case T2H_OP_DIV: return __fdiv_rn(x, y);
        case T2H_OP_RSUB: return sub_rn(y, x);
        default: return __fdiv_rn(y, x);
    }
}

template <typename T, int V>
__global__ __launch_bounds__(1024) void binop_kernel(EltArgs a) {
    Tile t;
    if (!tile_of<V>(a, t)) return;
    const T* __restrict__ x = static_cast<const T*>(a.x);
    T* __restrict__ o = static_cast<T*>(a.out);
    const BatchMap bm{a.batch.offsets, a.batch.rows_per_batch, a.batch.nbatch};
    const bool full = a.other_cols == a.cols;
    const int64_t ost = full ? a.p_stride : 1;
    float ov[V];
    int32_t cur = -1;
    float v[kRpt][V];
#pragma unroll
    for (int k = 0; k < kRpt; ++k) ld<T, V>(x + t.row(k) * a.cols + t.col0, v[k]);
#pragma unroll
    for (int k = 0; k < kRpt; ++k) {
        if (k >= t.nrows) break;
        const int64_t r = t.r0 + k;
        const int32_t b = bm.batch_of(r);
        if (b != cur) {
            if (full) {
                ldp<V>(a.gate + b * ost + t.col0, ov);
            } else {
                const float s = a.gate[b * ost];
#pragma unroll
                for (int i = 0; i < V; ++i) ov[i] = s;
            }
            cur = b;
        }
#pragma unroll
        for (int i = 0; i < V; ++i) v[k][i] = apply_op(v[k][i], ov[i], a.kind);
    }
    store_rows<T, V>(o, a.cols, t, v);
}

// ---- timestep embedding --------------------------------------------------------
struct FreqTable {
    float f[T2H_MAX_TIMESTEP_HALF];
};

template <typename T>
__global__ __launch_bounds__(kBlock) void timestep_kernel(const float* __restrict__ tv, T* __restrict__ out,
                                                          int64_t n, int32_t dim, FreqTable ft) {
    const int half = dim / 2;
    const int per_row = half + (dim & 1);
    const int64_t total = n * per_row;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
        const int64_t r = i / per_row;
        const int j = (int)(i % per_row);
        if (j >= half) {  // odd dim: zero last column
            st1(out + r * dim + dim - 1, 0.0f);
            continue;
        }
        const float angle = __fmul_rn(tv[r], ft.f[j]);
        float s, c;
        sincosf(angle, &s, &c);
        st1(out + r * dim + j, c);
        st1(out + r * dim + half + j, s);
    }
}

// ---- coords -> offsets ---------------------------------------------------------
__global__ void offsets_init_kernel(unsigned long long* first_bad) { *first_bad = 0x7FFFFFFFFFFFFFFFull; }

// Thread r (0 <= r <= rows) owns the batch boundaries between row r-1 and r:
// offsets[bb] = r for every bb in (b(r-1), b(r)], with b(-1) = -1 and
// b(rows) = nbatch. Rows of one batch are contiguous, so each offsets entry
// has exactly one writer when the coords are valid.
__global__ __launch_bounds__(kBlock) void offsets_kernel(const int32_t* __restrict__ coords, int64_t rows,
                                                         int32_t cc, int32_t nbatch, int64_t* __restrict__ offsets,
                                                         unsigned long long* first_bad) {
    for (int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x; r <= rows; r += (int64_t)gridDim.x * kBlock) {
        const int64_t prev = r > 0 ? (int64_t)coords[(r - 1) * cc] : -1;
        int64_t b;
        if (r < rows) {
            b = coords[r * cc];
            if (b < prev) {
                atomicMin(first_bad, (unsigned long long)((r << 1) | 0));
                continue;
            }
            if (b < 0 || b >= nbatch) {
                atomicMin(first_bad, (unsigned long long)((r << 1) | 1));
                continue;
            }
        } else {
            b = nbatch;
        }
        int64_t lo = prev + 1 < 0 ? 0 : prev + 1;
        int64_t hi = b > nbatch ? nbatch : b;
        for (int64_t bb = lo; bb <= hi; ++bb) offsets[bb] = r;
    }
}

__global__ __launch_bounds__(kBlock) void modulation_add_kernel(const float* __restrict__ mod,
                                                                const float* __restrict__ modulation,
                                                                float* __restrict__ m, int64_t n, int64_t width) {
    const int64_t total = n * width;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock)
        m[i] = add_rn(mod[i], modulation[i % width]);
}

// ---- launch helpers ------------------------------------------------------------
inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T>
bool vec_ok(const EltArgs& a) {
    constexpr int V = kPack<T>;
    return a.cols % V == 0 && al16(a.x) && al16(a.h) && al16(a.out) && al16(a.bias) && al16(a.gate) &&
           al16(a.shift) && a.p_stride % 4 == 0;
}

// Block width in threads: one row of 16-byte vectors when that is a whole
// number of waves (<= 1024 threads), else kBlock.
template <int V>
int tile_block(const EltArgs& a) {
    if (V > 1 && a.cols % (64 * V) == 0 && a.cols / V <= 1024) return a.cols / V;
    return kBlock;
}

// Launch a row-tiled kernel: 1-D grid of row tiles x column tiles, with the
// column-tile count set in the kernel's copy of the arguments.
template <int V, typename K>
hipError_t tile_launch(K kernel, EltArgs a, hipStream_t s) {
    const int64_t bw = (int64_t)tile_block<V>(a) * V;
    const int64_t rt = (a.rows + kRpt - 1) / kRpt;
    const int64_t ct = (a.cols + bw - 1) / bw;
    a.col_tiles = (int32_t)ct;
    a.fper = front_per(rt * ct);
    a.block_threads = tile_block<V>(a);
    hipLaunchKernelGGL(kernel, grid_1d(front_grid(rt * ct)), dim3(tile_block<V>(a)), 0, s, a);
    return hipGetLastError();
}

#define T2H_DISPATCH_DTYPE(DT, FN, ...)                                \
    switch (DT) {                                                      \
        case T2H_F32: return FN<float>(__VA_ARGS__);                   \
        case T2H_F16: return FN<_Float16>(__VA_ARGS__);                \
        default: return FN<__bf16>(__VA_ARGS__);                       \
    }

// The slab layout (act_slab_kernel) for 16-byte-aligned rows of at least one
// slab; row-tiled kernels for the rest.
template <typename T, int KIND, bool BIAS>
hipError_t act_launch(const EltArgs& a, hipStream_t s) {
    constexpr int V = kPack<T>;
    // column indices stay in int32: the last slab's lanes reach cols - 1 + 64 * V
    if (vec_ok<T>(a) && a.cols >= 64 * V && a.cols <= INT32_MAX - 64 * V) {
        const int64_t slabs = (a.cols + 64 * V - 1) / (64 * V);
        const int64_t tiles = (a.rows + kSlabRows - 1) / kSlabRows;
        // a dispatch counts work-items in 32 bits per grid dimension
        if (tiles < (int64_t(1) << 32) && slabs * kSlabThreads < (int64_t(1) << 32)) {
            const SlabArgs sa{a.x, a.out, a.bias, a.rows, a.cols};
            hipLaunchKernelGGL((act_slab_kernel<T, V, KIND, BIAS>), dim3((unsigned)slabs, (unsigned)tiles),
                               dim3(kSlabThreads), 0, s, sa);
            return hipGetLastError();
        }
    }
    if (vec_ok<T>(a)) return tile_launch<V>(act_kernel<T, V, KIND, BIAS>, a, s);
    return tile_launch<1>(act_kernel<T, 1, KIND, BIAS>, a, s);
}

template <typename T, int KIND>
hipError_t act_typed_kind(const EltArgs& a, hipStream_t s) {
    return a.bias ? act_launch<T, KIND, true>(a, s) : act_launch<T, KIND, false>(a, s);
}

template <typename T>
hipError_t act_typed(const EltArgs& a, hipStream_t s) {
    switch (a.kind) {
        case T2H_ACT_RELU: return act_typed_kind<T, T2H_ACT_RELU>(a, s);
        case T2H_ACT_SILU: return act_typed_kind<T, T2H_ACT_SILU>(a, s);
        case T2H_ACT_GELU: return act_typed_kind<T, T2H_ACT_GELU>(a, s);
        default: return act_typed_kind<T, T2H_ACT_GELU_TANH>(a, s);
    }
}

template <typename T>
hipError_t gate_res_typed(EltArgs a, hipStream_t s) {
    constexpr int V = kPack<T>;
    // the cached row loads address a row through a buffer descriptor: 32-bit byte offsets
    a.cached = a.rows * (int64_t)a.cols * (int64_t)sizeof(T) * 3 >= T2H_CACHED_SHARE_MIN &&
               (int64_t)a.cols * (int64_t)sizeof(T) <= INT32_MAX;
    if (vec_ok<T>(a)) return tile_launch<V>(gate_res_kernel<T, V>, a, s);
    return tile_launch<1>(gate_res_kernel<T, 1>, a, s);
}

template <typename T>
hipError_t modulate_typed(const EltArgs& a, hipStream_t s) {
    constexpr int V = kPack<T>;
    if (vec_ok<T>(a)) return tile_launch<V>(modulate_kernel<T, V>, a, s);
    return tile_launch<1>(modulate_kernel<T, 1>, a, s);
}

template <typename T>
hipError_t binop_typed(const EltArgs& a, hipStream_t s) {
    constexpr int V = kPack<T>;
    if (vec_ok<T>(a)) return tile_launch<V>(binop_kernel<T, V>, a, s);
    return tile_launch<1>(binop_kernel<T, 1>, a, s);
}

template <typename T>
hipError_t timestep_typed(const float* t, void* out, int64_t n, int32_t dim, const FreqTable& ft, hipStream_t s) {
    const int64_t total = n * (dim / 2 + (dim & 1));
    int64_t grid = (total + kBlock - 1) / kBlock;
    if (grid < 1) grid = 1;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(timestep_kernel<T>, dim3((unsigned)grid), dim3(kBlock), 0, s, t, static_cast<T*>(out), n, dim, ft);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_activation(const EltArgs& a, hipStream_t s) { T2H_DISPATCH_DTYPE(a.dtype, act_typed, a, s) }
hipError_t launch_gate_residual(const EltArgs& a, hipStream_t s) { T2H_DISPATCH_DTYPE(a.dtype, gate_res_typed, a, s) }
hipError_t launch_modulate(const EltArgs& a, hipStream_t s) { T2H_DISPATCH_DTYPE(a.dtype, modulate_typed, a, s) }
hipError_t launch_binop_rows(const EltArgs& a, hipStream_t s) { T2H_DISPATCH_DTYPE(a.dtype, binop_typed, a, s) }

hipError_t launch_timestep(const float* t, void* out, int64_t n, int32_t dim, int32_t dtype,
                           const float* freqs_host, hipStream_t s) {
    FreqTable ft{};
    for (int j = 0; j < dim / 2; ++j) ft.f[j] = freqs_host[j];
    T2H_DISPATCH_DTYPE(dtype, timestep_typed, t, out, n, dim, ft, s)
}

hipError_t launch_offsets(const int32_t* coords, int64_t rows, int32_t coord_cols, int32_t nbatch,
                          int64_t* offsets, int64_t* first_bad, hipStream_t s) {
    auto* fb = reinterpret_cast<unsigned long long*>(first_bad);
    hipLaunchKernelGGL(offsets_init_kernel, dim3(1), dim3(1), 0, s, fb);
    int64_t grid = (rows + 1 + kBlock - 1) / kBlock;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(offsets_kernel, dim3((unsigned)grid), dim3(kBlock), 0, s, coords, rows, coord_cols, nbatch,
                       offsets, fb);
    return hipGetLastError();
}

hipError_t launch_modulation_add(const float* mod, const float* modulation, float* m, int64_t n, int64_t width,
                                 hipStream_t s) {
    int64_t grid = (n * width + kBlock - 1) / kBlock;
    if (grid < 1) grid = 1;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(modulation_add_kernel, dim3((unsigned)grid), dim3(kBlock), 0, s, mod, modulation, m, n, width);
    return hipGetLastError();
}

}  // namespace t2h
