// C ABI of libt2h.so (declared in include/t2h.h): argument validation,
// thread-local error reporting, host-side tables (RoPE slots, timestep
// frequencies) and the synchronous host-pointer wrappers. Device entry points
// never allocate, synchronise or read device memory.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "t2h.h"
#include <cstdlib>

#include "t2h_internal.h"

namespace t2h {
namespace {

thread_local std::string g_last_error;

int32_t fail(int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int32_t ok() {
    g_last_error.clear();
    return T2H_OK;
}

int32_t hip_status(hipError_t e, const char* where) {
    if (e != hipSuccess) return fail(T2H_EHIP, "%s: %s", where, hipGetErrorString(e));
    return ok();
}

bool dtype_ok(int32_t dt) { return dt == T2H_F32 || dt == T2H_F16 || dt == T2H_BF16; }

int32_t check_batch(const int64_t* offsets, int32_t nbatch, int64_t rows_per_batch, const char* fn) {
    if (offsets != nullptr && nbatch < 1) return fail(T2H_EINVAL, "%s: offsets given with nbatch < 1", fn);
    if (rows_per_batch < 0) return fail(T2H_EINVAL, "%s: rows_per_batch < 0", fn);
    return T2H_OK;
}

// Highest batch index a row can map to (for parameter-array sizing checks the
// caller owns; we only reject impossible combinations here).
BatchArgs batch_args(const int64_t* offsets, int32_t nbatch, int64_t rows_per_batch) {
    BatchArgs b;
    b.offsets = offsets;
    b.nbatch = offsets ? nbatch : (nbatch > 0 ? nbatch : 1);
    b.rows_per_batch = offsets ? 0 : rows_per_batch;
    return b;
}

// Build the per-slot RoPE table from the caller's frequency table:
// slot p < pos_dim * freq_dim -> axis p / freq_dim, freq freqs[p % freq_dim]
// (modules/rope.mojo:51-60); other slots are identity.
int32_t build_slots(int32_t head_dim, const float* freqs_host, int32_t freq_dim, int32_t pos_dim,
                    RopeSlots& tab, const char* fn) {
    if (head_dim <= 0 || head_dim % 2 != 0) return fail(T2H_EINVAL, "%s: head_dim must be even and > 0", fn);
    const int half = head_dim / 2;
    if (half > T2H_MAX_HALF_HEAD) return fail(T2H_EUNSUPPORTED, "%s: head_dim > %d", fn, 2 * T2H_MAX_HALF_HEAD);
    if (pos_dim < 1 || pos_dim > T2H_MAX_POS_DIM) return fail(T2H_EINVAL, "%s: pos_dim must be in [1, %d]", fn, T2H_MAX_POS_DIM);
    if (freq_dim < 0 || (int64_t)freq_dim * pos_dim > half)
        return fail(T2H_EINVAL, "%s: freq_dim * pos_dim exceeds head_dim / 2", fn);
    if (freq_dim > 0 && freqs_host == nullptr) return fail(T2H_EINVAL, "%s: freqs_host is NULL", fn);
    std::memset(&tab, 0, sizeof(tab));
    for (int p = 0; p < T2H_MAX_HALF_HEAD; ++p) {
        if (p < half && p < pos_dim * freq_dim) {
            tab.axis[p] = (int8_t)(p / freq_dim);
            tab.freq[p] = freqs_host[p % freq_dim];
        } else {
            tab.axis[p] = -1;
            tab.freq[p] = 0.0f;
        }
    }
    return T2H_OK;
}

int32_t check_positions(const float* phases, int64_t phase_rows, const int32_t* coords, int32_t coord_cols,
                        int32_t grid_res, int32_t pos_dim, const char* fn) {
    if (phases != nullptr) {
        if (phase_rows <= 0) return fail(T2H_EINVAL, "%s: phase_rows must be > 0", fn);
        return T2H_OK;
    }
    if (coords != nullptr) {
        if (coord_cols < pos_dim + 1) return fail(T2H_EINVAL, "%s: coords must have pos_dim+1 columns", fn);
        return T2H_OK;
    }
    if (grid_res > 0) {
        if (pos_dim != 3) return fail(T2H_EINVAL, "%s: dense grid positions need pos_dim 3", fn);
        return T2H_OK;
    }
    return fail(T2H_EINVAL, "%s: RoPE needs phases, coords or grid_res", fn);
}

struct DeviceInfo {
    int cu = 0;
};
std::mutex g_dev_mu;
std::vector<DeviceInfo> g_dev;

}  // namespace

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if ((int)g_dev.size() <= dev) g_dev.resize(dev + 1);
    if (g_dev[dev].cu == 0) {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0) cu = 256;
        g_dev[dev].cu = cu;
    }
    return g_dev[dev].cu;
}

}  // namespace t2h

using namespace t2h;

extern "C" {

int32_t t2h_version(void) { return T2H_VERSION; }

const char* t2h_last_error(void) { return g_last_error.c_str(); }

int32_t t2h_device_init(int32_t device) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_status(e, "t2h_device_init");
    if (device < 0 || device >= n) return fail(T2H_EINVAL, "t2h_device_init: device %d of %d", device, n);
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_status(e, "t2h_device_init");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_status(e, "t2h_device_init");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(T2H_EDEVICE, "t2h_device_init: device %d is %s, libt2h is built for gfx950", device, prop.gcnArchName);
    (void)device_cu_count();
    double* scratch = nullptr;   // t2h_flow_euler_step_noalloc's scratch on this device
    e = euler_scratch(&scratch);
    if (e != hipSuccess) return hip_status(e, "t2h_device_init");
    return ok();
}

int32_t t2h_ln_modulate(const void* x, void* out, int64_t rows, int32_t cols, int32_t dtype, float eps, int32_t mode,
                        const float* p0, const float* p1, int64_t p_stride, const int64_t* offsets, int32_t nbatch,
                        int64_t rows_per_batch, void* stream) {
    const char* fn = "t2h_ln_modulate";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape [%lld, %d]", fn, (long long)rows, cols);
    if (mode < T2H_LN_PLAIN || mode > T2H_LN_AFFINE) return fail(T2H_EINVAL, "%s: bad mode %d", fn, mode);
    if (mode != T2H_LN_PLAIN && (p0 == nullptr || p1 == nullptr)) return fail(T2H_EINVAL, "%s: mode %d needs p0 and p1", fn, mode);
    if (p_stride != 0 && p_stride < cols) return fail(T2H_EINVAL, "%s: p_stride < cols", fn);
    if (!(eps >= 0.0f)) return fail(T2H_EINVAL, "%s: eps must be >= 0", fn);
    if (int32_t rc = check_batch(offsets, nbatch, rows_per_batch, fn)) return rc;
    if (rows == 0) return ok();
    if (x == nullptr || out == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    LnArgs a{};
    a.x = x;
    a.y_out = out;
    a.eps = eps;
    a.mode = mode;
    a.p0 = p0;
    a.p1 = p1;
    a.p_stride = p_stride ? p_stride : cols;
    a.rows = rows;
    a.cols = cols;
    a.dtype = dtype;
    a.batch = batch_args(offsets, nbatch, rows_per_batch);
    return hip_status(launch_ln(a, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_gate_residual_ln_modulate(const void* x, const void* h, void* x_out, void* y_out, const float* bias,
                                      const float* gate, int64_t gate_stride, float eps, int32_t mode, const float* p0,
                                      const float* p1, int64_t p_stride, int64_t rows, int32_t cols, int32_t dtype,
                                      const int64_t* offsets, int32_t nbatch, int64_t rows_per_batch, void* stream) {
    const char* fn = "t2h_gate_residual_ln_modulate";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (mode < T2H_LN_PLAIN || mode > T2H_LN_AFFINE) return fail(T2H_EINVAL, "%s: bad mode %d", fn, mode);
    if (mode != T2H_LN_PLAIN && (p0 == nullptr || p1 == nullptr)) return fail(T2H_EINVAL, "%s: mode %d needs p0 and p1", fn, mode);
    if ((p_stride != 0 && p_stride < cols) || (gate_stride != 0 && gate_stride < cols))
        return fail(T2H_EINVAL, "%s: parameter stride < cols", fn);
    if (!(eps >= 0.0f)) return fail(T2H_EINVAL, "%s: eps must be >= 0", fn);
    if (int32_t rc = check_batch(offsets, nbatch, rows_per_batch, fn)) return rc;
    if (rows == 0) return ok();
    if (x == nullptr || h == nullptr || x_out == nullptr || y_out == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    if (y_out == x || y_out == h || y_out == x_out) return fail(T2H_EINVAL, "%s: y_out must not alias x, h or x_out", fn);
    LnArgs a{};
    a.x = x;
    a.h = h;
    a.x_out = x_out;
    a.y_out = y_out;
    a.bias = bias;
    a.gate = gate;
    a.gate_stride = gate_stride ? gate_stride : cols;
    a.eps = eps;
    a.mode = mode;
    a.p0 = p0;
    a.p1 = p1;
    a.p_stride = p_stride ? p_stride : cols;
    a.rows = rows;
    a.cols = cols;
    a.dtype = dtype;
    a.batch = batch_args(offsets, nbatch, rows_per_batch);
    return hip_status(launch_ln(a, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_modulate(const void* x, void* out, int64_t rows, int32_t cols, int32_t dtype, const float* shift,
                     const float* scale, int64_t p_stride, const int64_t* offsets, int32_t nbatch,
                     int64_t rows_per_batch, void* stream) {
    const char* fn = "t2h_modulate";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (shift == nullptr || scale == nullptr) return fail(T2H_EINVAL, "%s: shift/scale NULL", fn);
    if (p_stride != 0 && p_stride < cols) return fail(T2H_EINVAL, "%s: p_stride < cols", fn);
    if (int32_t rc = check_batch(offsets, nbatch, rows_per_batch, fn)) return rc;
    if (rows == 0) return ok();
    if (x == nullptr || out == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    EltArgs a{};
    a.x = x;
    a.out = out;
    a.gate = scale;
    a.shift = shift;
    a.p_stride = p_stride ? p_stride : cols;
    a.rows = rows;
    a.cols = cols;
    a.dtype = dtype;
    a.batch = batch_args(offsets, nbatch, rows_per_batch);
    return hip_status(launch_modulate(a, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_binop_rows(const void* x, const float* other, void* out, int64_t rows, int32_t cols, int32_t other_cols,
                       int32_t dtype, int32_t op, const int64_t* offsets, int32_t nbatch, int64_t rows_per_batch,
                       void* stream) {
    const char* fn = "t2h_binop_rows";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (other_cols != cols && other_cols != 1) return fail(T2H_EINVAL, "Tensor._binop_rows: incompatible row size");
    if (op < T2H_OP_ADD || op > T2H_OP_RDIV) return fail(T2H_EINVAL, "%s: bad op %d", fn, op);
    if (int32_t rc = check_batch(offsets, nbatch, rows_per_batch, fn)) return rc;
    if (rows == 0) return ok();
    if (x == nullptr || out == nullptr || other == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    EltArgs a{};
    a.x = x;
    a.out = out;
    a.gate = other;
    a.p_stride = other_cols;
    a.rows = rows;
    a.cols = cols;
    a.other_cols = other_cols;
    a.dtype = dtype;
    a.kind = op;
    a.batch = batch_args(offsets, nbatch, rows_per_batch);
    return hip_status(launch_binop_rows(a, static_cast<hipStream_t>(stream)), fn);
}

static int32_t qk_common(const void* q_in, const void* k_in, void* q_out, void* k_out, void* v, int64_t rows,
                         int64_t in_stride, int64_t out_stride, int32_t heads, int32_t head_dim, int32_t dtype,
                         const float* bias_q, const float* bias_k, const float* bias_v, const float* gamma_q,
                         const float* gamma_k, int32_t use_rope, const float* freqs_host, int32_t freq_dim,
                         int32_t pos_dim, const float* phases, int64_t phase_rows, const int32_t* coords,
                         int32_t coord_cols, int32_t grid_res, void* stream, const char* fn) {
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows < 0 || heads <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    const int64_t hd = (int64_t)heads * head_dim;
    if (in_stride == 0) in_stride = hd;
    if (out_stride == 0) out_stride = hd;
    if (in_stride < hd || out_stride < hd) return fail(T2H_EINVAL, "%s: row stride < heads * head_dim", fn);
    RopeSlots tab;
    if (use_rope) {
        if (int32_t rc = build_slots(head_dim, freqs_host, freq_dim, pos_dim, tab, fn)) return rc;
        if (int32_t rc = check_positions(phases, phase_rows, coords, coord_cols, grid_res, pos_dim, fn)) return rc;
    } else {
        if (head_dim <= 0 || head_dim % 2 != 0) return fail(T2H_EINVAL, "%s: head_dim must be even and > 0", fn);
        if (head_dim / 2 > T2H_MAX_HALF_HEAD) return fail(T2H_EUNSUPPORTED, "%s: head_dim too large", fn);
        std::memset(&tab, 0, sizeof(tab));
    }
    if ((gamma_q == nullptr) != (gamma_k == nullptr) && q_in != nullptr && k_in != nullptr)
        return fail(T2H_EINVAL, "%s: gamma_q and gamma_k must both be given or both NULL", fn);
    if (rows == 0) return ok();
    if (q_in == nullptr && k_in == nullptr) return fail(T2H_EINVAL, "%s: q and k are both NULL", fn);
    if ((q_in != nullptr) != (q_out != nullptr) || (k_in != nullptr) != (k_out != nullptr))
        return fail(T2H_EINVAL, "%s: input/output pointer mismatch", fn);
    QkArgs a{};
    a.q_in = q_in;
    a.k_in = k_in;
    a.q_out = q_out;
    a.k_out = k_out;
    a.v = v;
    a.rows = rows;
    a.in_stride = in_stride;
    a.out_stride = out_stride;
    a.heads = heads;
    a.head_dim = head_dim;
    a.dtype = dtype;
    a.bias_q = bias_q;
    a.bias_k = bias_k;
    a.bias_v = bias_v;
    a.gamma_q = gamma_q;
    a.gamma_k = gamma_k;
    a.rms_scale = (float)std::pow((double)head_dim, 0.5);  // Float32(Float64(dim) ** 0.5)
    a.use_rope = use_rope ? 1 : 0;
    a.pos_dim = pos_dim;
    a.freq_dim = use_rope ? freq_dim : 0;
    a.phases = use_rope ? phases : nullptr;
    a.phase_rows = phase_rows;
    a.coords = (use_rope && phases == nullptr) ? coords : nullptr;
    a.coord_cols = coord_cols;
    a.grid_res = grid_res;
    return hip_status(launch_qk(a, tab, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_qk_rmsnorm_rope(const void* q_in, const void* k_in, void* q_out, void* k_out, int64_t rows,
                            int64_t in_stride, int64_t out_stride, int32_t heads, int32_t head_dim, int32_t dtype,
                            const float* bias_q, const float* bias_k, const float* gamma_q, const float* gamma_k,
                            int32_t use_rope, const float* freqs_host, int32_t freq_dim, int32_t pos_dim,
                            const float* phases, int64_t phase_rows, const int32_t* coords, int32_t coord_cols,
                            int32_t grid_res, void* stream) {
    return qk_common(q_in, k_in, q_out, k_out, nullptr, rows, in_stride, out_stride, heads, head_dim, dtype, bias_q,
                     bias_k, nullptr, gamma_q, gamma_k, use_rope, freqs_host, freq_dim, pos_dim, phases, phase_rows,
                     coords, coord_cols, grid_res, stream, "t2h_qk_rmsnorm_rope");
}

int32_t t2h_qkv_bias_rmsnorm_rope(void* qkv, int64_t rows, int32_t heads, int32_t head_dim, int32_t dtype,
                                  const float* bias, const float* gamma_q, const float* gamma_k, int32_t use_rope,
                                  const float* freqs_host, int32_t freq_dim, int32_t pos_dim, const float* phases,
                                  int64_t phase_rows, const int32_t* coords, int32_t coord_cols, int32_t grid_res,
                                  void* stream) {
    const char* fn = "t2h_qkv_bias_rmsnorm_rope";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows > 0 && qkv == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    const int64_t hd = (int64_t)heads * head_dim;
    const size_t es = dtype == T2H_F32 ? 4 : 2;
    char* base = static_cast<char*>(qkv);
    void* k = base ? base + hd * es : nullptr;
    void* v = base ? base + 2 * hd * es : nullptr;
    return qk_common(qkv, k, qkv, k, bias ? v : nullptr, rows, 3 * hd, 3 * hd, heads, head_dim, dtype, bias,
                     bias ? bias + hd : nullptr, bias ? bias + 2 * hd : nullptr, gamma_q, gamma_k, use_rope,
                     freqs_host, freq_dim, pos_dim, phases, phase_rows, coords, coord_cols, grid_res, stream, fn);
}

static bool aligned(const void* p, int64_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

int32_t t2h_attn_pack(const void* q, const void* k, const void* v, int64_t in_stride, int64_t rows, int32_t heads,
                      int32_t head_dim, int32_t dtype, const float* bias_q, const float* bias_k, const float* bias_v,
                      const float* gamma_q, const float* gamma_k, int32_t use_rope, const float* freqs_host,
                      int32_t freq_dim, int32_t pos_dim, const float* phases, int64_t phase_rows,
                      const int32_t* coords, int32_t coord_cols, int32_t grid_res, void* qh, int64_t mp, void* k_out,
                      void* vh, int64_t lp, int32_t k_transposed, void* stream) {
    const char* fn = "t2h_attn_pack";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows < 0 || heads <= 0 || heads > 65535) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (head_dim != 64 && head_dim != 128) return fail(T2H_EUNSUPPORTED, "%s: head_dim must be 64 or 128", fn);
    const int64_t hd = (int64_t)heads * head_dim;
    if (in_stride == 0) in_stride = hd;
    if (in_stride < hd) return fail(T2H_EINVAL, "%s: row stride < heads * head_dim", fn);
    if (qh == nullptr && k_out == nullptr && vh == nullptr) return fail(T2H_EINVAL, "%s: no output", fn);
    if (rows > 0 && ((qh != nullptr && q == nullptr) || (k_out != nullptr && k == nullptr) ||
                     (vh != nullptr && v == nullptr)))
        return fail(T2H_EINVAL, "%s: an output needs its input tensor", fn);
    if (qh != nullptr && mp < rows) return fail(T2H_EINVAL, "%s: mp < rows", fn);
    if ((k_out != nullptr || vh != nullptr) && lp < rows) return fail(T2H_EINVAL, "%s: lp < rows", fn);
    if (k_out != nullptr && k_transposed && lp % 8 != 0) return fail(T2H_EINVAL, "%s: transposed k needs lp %% 8 == 0", fn);
    if (qh == nullptr) mp = 0;
    if (k_out == nullptr && vh == nullptr) lp = 0;
    if (qh != nullptr && k_out != nullptr && (gamma_q == nullptr) != (gamma_k == nullptr))
        return fail(T2H_EINVAL, "%s: gamma_q and gamma_k must both be given or both NULL", fn);
    RopeSlots tab;
    std::memset(&tab, 0, sizeof(tab));
    if (use_rope && (qh != nullptr || k_out != nullptr)) {
        if (int32_t rc = build_slots(head_dim, freqs_host, freq_dim, pos_dim, tab, fn)) return rc;
        if (int32_t rc = check_positions(phases, phase_rows, coords, coord_cols, grid_res, pos_dim, fn)) return rc;
    } else {
        use_rope = 0;
    }
    // each lane moves head_dim/16 elements: min(16, that many bytes) alignment
    const int64_t es = dtype == T2H_F32 ? 4 : 2;
    const int64_t chunk = (head_dim / 16) * es < 16 ? (head_dim / 16) * es : 16;
    if ((in_stride * es) % chunk != 0 || !aligned(q, chunk) || !aligned(k, chunk) || !aligned(v, chunk))
        return fail(T2H_EINVAL, "%s: inputs must be %lld-byte aligned", fn, (long long)chunk);
    if (!aligned(qh, 16) || !aligned(k_out, 16) || !aligned(vh, 16) || !aligned(bias_q, 16) || !aligned(bias_k, 16) ||
        !aligned(bias_v, 16) || !aligned(gamma_q, 16) || !aligned(gamma_k, 16) || !aligned(phases, 16))
        return fail(T2H_EINVAL, "%s: outputs and f32 parameters must be 16-byte aligned", fn);
    if (mp == 0 && lp == 0) return ok();
    PackArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.rows = rows;
    a.in_stride = in_stride;
    a.heads = heads;
    a.head_dim = head_dim;
    a.dtype = dtype;
    a.bias_q = bias_q;
    a.bias_k = bias_k;
    a.bias_v = bias_v;
    a.gamma_q = gamma_q;
    a.gamma_k = gamma_k;
    a.rms_scale = std::sqrt((float)head_dim);           // sqrt(Float32(d)), attention.mojo:539
    a.q_scale = 1.0f / std::sqrt((float)head_dim);      // attention.mojo:587
    a.use_rope = use_rope ? 1 : 0;
    a.pos_dim = pos_dim;
    a.phases = use_rope ? phases : nullptr;
    a.phase_rows = phase_rows;
    a.coords = (use_rope && phases == nullptr) ? coords : nullptr;
    a.coord_cols = coord_cols;
    a.grid_res = grid_res;
    a.qh = qh;
    a.mp = mp;
    a.k_out = k_out;
    a.vh = vh;
    a.lp = lp;
    a.k_transposed = k_transposed ? 1 : 0;
    return hip_status(launch_pack(a, tab, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_qkv_linear_pack(const void* x, int64_t ldx, const void* w, int64_t rows, int32_t in_features,
                            int32_t heads, int32_t head_dim, int32_t dtype, const float* bias_q, const float* bias_k,
                            const float* bias_v, const float* gamma_q, const float* gamma_k, int32_t use_rope,
                            const float* freqs_host, int32_t freq_dim, int32_t pos_dim, const float* phases,
                            int64_t phase_rows, const int32_t* coords, int32_t coord_cols, int32_t grid_res,
                            void* qh, int64_t mp, void* k_out, void* vh, int64_t lp, int32_t k_transposed,
                            void* stream) {
    const char* fn = "t2h_qkv_linear_pack";
    if (dtype != T2H_F16 && dtype != T2H_BF16) return fail(T2H_EINVAL, "%s: operands must be f16 or bf16", fn);
    if (rows < 0 || heads <= 0 || heads > 65535 || in_features <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (!gemm_head_dim_ok(head_dim)) return fail(T2H_EUNSUPPORTED, "%s: head_dim must be 64 or 128", fn);
    const int64_t n = 3 * (int64_t)heads * head_dim;
    // whole feature tiles, each wave's 128 features inside one tensor
    if (n % gemm_feature_tile() != 0 || ((int64_t)heads * head_dim) % 128 != 0 || n > INT32_MAX)
        return fail(T2H_EUNSUPPORTED, "%s: 3 * heads * head_dim must be a multiple of %d (heads: even for "
                    "head_dim 128, a multiple of 4 for 64)", fn, gemm_feature_tile());
    if (in_features % gemm_k_step() != 0)
        return fail(T2H_EINVAL, "%s: in_features %d is not a multiple of %d", fn, in_features, gemm_k_step());
    if (ldx < in_features || ldx % 8 != 0) return fail(T2H_EINVAL, "%s: ldx must be >= in_features and a multiple of 8", fn);
    if (qh == nullptr || k_out == nullptr || vh == nullptr) return fail(T2H_EINVAL, "%s: NULL output", fn);
    if (mp < rows || lp < rows) return fail(T2H_EINVAL, "%s: mp and lp must be >= rows", fn);
    if (k_transposed && lp % 8 != 0) return fail(T2H_EINVAL, "%s: transposed k needs lp %% 8 == 0", fn);
    if ((gamma_q == nullptr) != (gamma_k == nullptr))
        return fail(T2H_EINVAL, "%s: gamma_q and gamma_k must both be given or both NULL", fn);
    RopeSlots tab;
    std::memset(&tab, 0, sizeof(tab));
    if (use_rope) {
        if (int32_t rc = build_slots(head_dim, freqs_host, freq_dim, pos_dim, tab, fn)) return rc;
        if (int32_t rc = check_positions(phases, phase_rows, coords, coord_cols, grid_res, pos_dim, fn)) return rc;
    }
    if (rows > 0 && (x == nullptr || w == nullptr)) return fail(T2H_EINVAL, "%s: NULL input", fn);
    if (!aligned(x, 16) || !aligned(w, 16) || !aligned(qh, 16) || !aligned(k_out, 16) || !aligned(vh, 16) ||
        !aligned(bias_q, 16) || !aligned(bias_k, 16) || !aligned(bias_v, 16) || !aligned(gamma_q, 16) ||
        !aligned(gamma_k, 16) || !aligned(phases, 16))
        return fail(T2H_EINVAL, "%s: tensors and f32 parameters must be 16-byte aligned", fn);
    if (mp == 0 && lp == 0) return ok();
    GemmArgs g{};
    g.x = x;
    g.ldx = ldx;
    g.w = w;
    g.rows = rows;
    g.n = (int32_t)n;
    g.k = in_features;
    g.dtype = dtype;
    PackArgs a{};
    a.rows = rows;
    a.heads = heads;
    a.head_dim = head_dim;
    a.dtype = dtype;
    a.bias_q = bias_q;
    a.bias_k = bias_k;
    a.bias_v = bias_v;
    a.gamma_q = gamma_q;
    a.gamma_k = gamma_k;
    a.rms_scale = std::sqrt((float)head_dim);           // sqrt(Float32(d)), attention.mojo:539
    a.q_scale = 1.0f / std::sqrt((float)head_dim);      // attention.mojo:587
    a.use_rope = use_rope ? 1 : 0;
    a.pos_dim = pos_dim;
    a.phases = use_rope ? phases : nullptr;
    a.phase_rows = phase_rows;
    a.coords = (use_rope && phases == nullptr) ? coords : nullptr;
    a.coord_cols = coord_cols;
    a.grid_res = grid_res;
    a.qh = qh;
    a.mp = mp;
    a.k_out = k_out;
    a.vh = vh;
    a.lp = lp;
    a.k_transposed = k_transposed ? 1 : 0;
    return hip_status(launch_qkv_pack(g, a, tab, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_rope_freqs(int32_t head_dim, int32_t dim, double freq_lo, double freq_hi, float* freqs_host,
                       int32_t capacity) {
    if (head_dim <= 0 || head_dim % 2 != 0)
        return fail(T2H_EINVAL, "RotaryPositionEmbedder: head_dim must be even");
    if (dim <= 0) return fail(T2H_EINVAL, "t2h_rope_freqs: dim must be > 0");
    const int32_t fd = head_dim / 2 / dim;
    for (int32_t j = 0; j < fd && j < capacity; ++j) {
        const float e = (float)j / (float)fd;
        freqs_host[j] = (float)freq_lo / std::pow((float)freq_hi, e);   // powf, as the constructor's f32 **
    }
    ok();
    return fd;
}

int32_t t2h_rope_phases(float* phases_out, int64_t rows, int32_t head_dim, const float* freqs_host, int32_t freq_dim,
                        int32_t pos_dim, const float* positions, const int32_t* coords, int32_t coord_cols,
                        int32_t grid_res, void* stream) {
    const char* fn = "t2h_rope_phases";
    if (rows < 0) return fail(T2H_EINVAL, "%s: rows < 0", fn);
    RopeSlots tab;
    if (int32_t rc = build_slots(head_dim, freqs_host, freq_dim, pos_dim, tab, fn)) return rc;
    if (positions == nullptr)
        if (int32_t rc = check_positions(nullptr, 0, coords, coord_cols, grid_res, pos_dim, fn)) return rc;
    if (rows == 0) return ok();
    if (phases_out == nullptr) return fail(T2H_EINVAL, "%s: NULL output", fn);
    PhaseArgs a{};
    a.out = phases_out;
    a.rows = rows;
    a.head_dim = head_dim;
    a.pos_dim = pos_dim;
    a.positions = positions;
    a.coords = positions ? nullptr : coords;
    a.coord_cols = coord_cols;
    a.grid_res = grid_res;
    return hip_status(launch_phases(a, tab, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_activation(const void* x, void* out, const float* bias, int64_t rows, int32_t cols, int32_t dtype,
                       int32_t kind, void* stream) {
    const char* fn = "t2h_activation";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (kind < T2H_ACT_RELU || kind > T2H_ACT_GELU_TANH) return fail(T2H_EINVAL, "unknown activation");
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (rows == 0) return ok();
    if (x == nullptr || out == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    EltArgs a{};
    a.x = x;
    a.out = out;
    a.bias = bias;
    a.rows = rows;
    a.cols = cols;
    a.dtype = dtype;
    a.kind = kind;
    return hip_status(launch_activation(a, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_linear(const void* x, int64_t ldx, const void* w, const float* bias, void* out, int64_t ldo, int64_t rows,
                   int32_t in_features, int32_t out_features, int32_t dtype, int32_t out_dtype, int32_t act,
                   void* stream) {
    const char* fn = "t2h_linear";
    if (dtype != T2H_F16 && dtype != T2H_BF16) return fail(T2H_EINVAL, "%s: operands must be f16 or bf16", fn);
    if (out_dtype != T2H_F32 && out_dtype != dtype)
        return fail(T2H_EINVAL, "%s: out_dtype must be f32 or the operand dtype", fn);
    if (act != T2H_ACT_NONE && (act < T2H_ACT_RELU || act > T2H_ACT_GELU_TANH))
        return fail(T2H_EINVAL, "unknown activation");
    if (rows < 0 || in_features <= 0 || out_features <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (out_features % gemm_feature_tile() != 0)
        return fail(T2H_EINVAL, "%s: out_features %d is not a multiple of %d", fn, out_features, gemm_feature_tile());
    if (in_features % gemm_k_step() != 0)
        return fail(T2H_EINVAL, "%s: in_features %d is not a multiple of %d", fn, in_features, gemm_k_step());
    if (ldx < in_features || ldo < out_features) return fail(T2H_EINVAL, "%s: row stride below the row", fn);
    if (ldx % 8 != 0 || ldo % (out_dtype == T2H_F32 ? 4 : 8) != 0)
        return fail(T2H_EINVAL, "%s: ldx must be a multiple of 8, ldo of %d", fn, out_dtype == T2H_F32 ? 4 : 8);
    if (rows == 0) return ok();
    if (x == nullptr || w == nullptr || out == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    if (!aligned(x, 16) || !aligned(w, 16) || (bias != nullptr && !aligned(bias, 16)) ||
        !aligned(out, 16))
        return fail(T2H_EINVAL, "%s: misaligned tensor", fn);
    GemmArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.w = w;
    a.rows = rows;
    a.n = out_features;
    a.k = in_features;
    a.dtype = dtype;
    a.bias = bias;
    a.act = act;
    a.out = out;
    a.ldo = ldo;
    a.out_dtype = out_dtype;
    return hip_status(launch_gemm(a, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_linear_gate_residual(const void* x, int64_t ldx, const void* w, const float* bias, const void* res,
                                 void* out, int64_t ldo, int64_t rows, int32_t in_features, int32_t out_features,
                                 int32_t dtype, int32_t out_dtype, const float* gate, int64_t gate_stride,
                                 const int64_t* offsets, int32_t nbatch, int64_t rows_per_batch, void* stream) {
    const char* fn = "t2h_linear_gate_residual";
    if (dtype != T2H_F16 && dtype != T2H_BF16) return fail(T2H_EINVAL, "%s: operands must be f16 or bf16", fn);
    if (out_dtype != T2H_F32 && out_dtype != dtype)
        return fail(T2H_EINVAL, "%s: out_dtype must be f32 or the operand dtype", fn);
    if (rows < 0 || in_features <= 0 || out_features <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (out_features % gemm_feature_tile() != 0)
        return fail(T2H_EINVAL, "%s: out_features %d is not a multiple of %d", fn, out_features, gemm_feature_tile());
    if (in_features % gemm_k_step() != 0)
        return fail(T2H_EINVAL, "%s: in_features %d is not a multiple of %d", fn, in_features, gemm_k_step());
    if (ldx < in_features || ldo < out_features) return fail(T2H_EINVAL, "%s: row stride below the row", fn);
    if (ldx % 8 != 0 || ldo % (out_dtype == T2H_F32 ? 4 : 8) != 0)
        return fail(T2H_EINVAL, "%s: ldx must be a multiple of 8, ldo of %d", fn, out_dtype == T2H_F32 ? 4 : 8);
    if (gate != nullptr && gate_stride == 0) gate_stride = out_features;
    if (gate != nullptr && gate_stride < out_features) return fail(T2H_EINVAL, "%s: gate_stride < out_features", fn);
    if (int32_t rc = check_batch(offsets, nbatch, rows_per_batch, fn)) return rc;
    if (rows == 0) return ok();
    if (x == nullptr || w == nullptr || res == nullptr || out == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    if (!aligned(x, 16) || !aligned(w, 16) || !aligned(res, 16) || !aligned(out, 16) ||
        (bias != nullptr && !aligned(bias, 16)) || (gate != nullptr && (!aligned(gate, 16) || gate_stride % 4 != 0)))
        return fail(T2H_EINVAL, "%s: misaligned tensor", fn);
    GemmArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.w = w;
    a.rows = rows;
    a.n = out_features;
    a.k = in_features;
    a.dtype = dtype;
    a.bias = bias;
    a.act = T2H_ACT_NONE;
    a.out = out;
    a.ldo = ldo;
    a.out_dtype = out_dtype;
    a.res = res;
    a.gate = gate;
    a.gate_stride = gate_stride;
    a.batch = BatchArgs{offsets, gate != nullptr ? nbatch : 0, rows_per_batch};
    return hip_status(launch_gemm_residual(a, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_gate_residual(const void* x, const void* h, void* out, const float* bias, const float* gate,
                          int64_t p_stride, int64_t rows, int32_t cols, int32_t dtype, const int64_t* offsets,
                          int32_t nbatch, int64_t rows_per_batch, void* stream) {
    const char* fn = "t2h_gate_residual";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (p_stride != 0 && p_stride < cols) return fail(T2H_EINVAL, "%s: p_stride < cols", fn);
    if (int32_t rc = check_batch(offsets, nbatch, rows_per_batch, fn)) return rc;
    if (rows == 0) return ok();
    if (h == nullptr || out == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    EltArgs a{};
    a.x = x;
    a.h = h;
    a.out = out;
    a.bias = bias;
    a.gate = gate;
    a.p_stride = p_stride ? p_stride : cols;
    a.rows = rows;
    a.cols = cols;
    a.dtype = dtype;
    a.batch = batch_args(offsets, nbatch, rows_per_batch);
    return hip_status(launch_gate_residual(a, static_cast<hipStream_t>(stream)), fn);
}

// Host frequency table of the timestep embedding, in the reference's f32
// order: neg_log = -f32(log(f64 max_period)); freq_j = exp(neg_log * j / half)
// (models/sparse_structure_flow.mojo:69-72).
static void timestep_freqs(int32_t dim, double max_period, float* f) {
    const int half = dim / 2;
    const float neg_log = -(float)std::log(max_period);
    for (int j = 0; j < half; ++j) {
        const float num = neg_log * (float)j;
        f[j] = std::exp(num / (float)half);
    }
}

int32_t t2h_timestep_embedding(const float* t, void* out, int64_t n, int32_t dim, int32_t dtype, double max_period,
                               void* stream) {
    const char* fn = "t2h_timestep_embedding";
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (n < 0 || dim <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (dim / 2 > T2H_MAX_TIMESTEP_HALF) return fail(T2H_EUNSUPPORTED, "%s: dim / 2 > %d", fn, T2H_MAX_TIMESTEP_HALF);
    if (!(max_period > 0.0)) return fail(T2H_EINVAL, "%s: max_period must be > 0", fn);
    if (n == 0) return ok();
    if (t == nullptr || out == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    float freqs[T2H_MAX_TIMESTEP_HALF];
    timestep_freqs(dim, max_period, freqs);
    return hip_status(launch_timestep(t, out, n, dim, dtype, freqs, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_coords_to_offsets(const int32_t* coords, int64_t rows, int32_t coord_cols, int32_t nbatch,
                              int64_t* offsets, int64_t* first_bad, void* stream) {
    const char* fn = "t2h_coords_to_offsets";
    if (rows < 0 || coord_cols < 1 || nbatch < 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (offsets == nullptr || first_bad == nullptr) return fail(T2H_EINVAL, "%s: NULL output", fn);
    if (rows > 0 && coords == nullptr) return fail(T2H_EINVAL, "%s: NULL coords", fn);
    if (rows >= (int64_t(1) << 62)) return fail(T2H_EINVAL, "%s: too many rows", fn);
    return hip_status(launch_offsets(coords, rows, coord_cols, nbatch, offsets, first_bad,
                                     static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_modulation_add(const float* mod, const float* modulation, float* m, int64_t n, int64_t width,
                           void* stream) {
    const char* fn = "t2h_modulation_add";
    if (n < 0 || width <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (n == 0) return ok();
    if (mod == nullptr || modulation == nullptr || m == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    return hip_status(launch_modulation_add(mod, modulation, m, n, width, static_cast<hipStream_t>(stream)), fn);
}

// Flow-matching Euler step. The rescale's workspace holds the statistics
// pass's f64 partial quads [nstats][4]: at most kStatsMaxPerSeg per segment.
static int64_t stats_blocks(int64_t m) {
    const int64_t c = (m + kStatsMinShare - 1) / kStatsMinShare;
    return c < kStatsMaxPerSeg ? c : kStatsMaxPerSeg;
}

int64_t t2h_flow_euler_workspace(int64_t rows, int64_t row_size, int32_t n_seg_offsets) {
    if (rows < 0 || row_size < 0 || n_seg_offsets < 0) return -1;
    int64_t blocks;
    if (n_seg_offsets > 0) {   // segment sizes unknown here: the largest total over any split
        const int64_t nseg = n_seg_offsets - 1;
        const int64_t a = nseg * (int64_t)kStatsMaxPerSeg;
        const int64_t b = (rows * row_size + kStatsMinShare - 1) / kStatsMinShare + nseg;
        blocks = a < b ? a : b;
    } else {
        blocks = rows * stats_blocks(row_size);
    }
    // one segment: room for the one-launch form (barrier words + partials)
    const bool one_seg = n_seg_offsets == 2 || (n_seg_offsets == 0 && rows == 1);
    return one_seg && blocks * 32 < kFuseBytes ? kFuseBytes : blocks * 32;
}

// Polls a data block of the one-launch rescale waits for the ratio before it
// leaves its vectors to the reducing block (a normal wait takes tens). The
// environment's T2H_FUSE_WAIT_POLLS overrides it, read on every call: 0
// makes every block leave, which the tests use to run that path.
static int32_t fuse_wait_polls() {
    const char* e = std::getenv("T2H_FUSE_WAIT_POLLS");
    if (e == nullptr || *e == '\0') return 1 << 12;
    const long v = std::strtol(e, nullptr, 10);
    return v < 0 ? 0 : (v > (1 << 20) ? (1 << 20) : (int32_t)v);
}

// builtin: the statistics go to the library's per-device scratch instead of
// the caller's workspace (t2h_flow_euler_step_noalloc).
static int32_t euler_step(const void* x_t, const void* v_pos, const void* v_neg, void* x_prev, void* pred_x0,
                          int64_t rows, int64_t row_size, int32_t dtype, double t, double t_prev, double sigma_min,
                          double guidance_strength, double guidance_rescale, const int64_t* seg_offsets_host,
                          int32_t n_seg_offsets, void* workspace, int64_t workspace_bytes, bool builtin,
                          void* stream, const char* fn) {
    if (!dtype_ok(dtype)) return fail(T2H_EINVAL, "%s: bad dtype %d", fn, dtype);
    if (rows < 0 || row_size <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    if (n_seg_offsets < 0 || n_seg_offsets == 1) return fail(T2H_EINVAL, "%s: seg_offsets needs >= 2 entries", fn);
    const int64_t n = rows * row_size;
    if (n == 0) return ok();
    if (x_t == nullptr || v_pos == nullptr || x_prev == nullptr) return fail(T2H_EINVAL, "%s: NULL tensor", fn);
    EulerArgs a{};
    a.x = x_t;
    a.v_pos = v_pos;
    a.v_neg = v_neg;
    a.x_prev = x_prev;
    a.pred_x0 = pred_x0;
    a.n = n;
    a.row_size = row_size;
    a.dtype = dtype;
    // _inference (flow_euler.mojo:167-181): strength 1 -> the positive
    // prediction alone, 0 -> the negative alone, neither is rescaled
    a.mode = 0;
    if (v_neg != nullptr) {
        if (guidance_strength == 0.0) a.v_pos = v_neg;
        else if (guidance_strength != 1.0) a.mode = guidance_rescale > 0.0 ? 2 : 1;
    }
    a.gp = (float)guidance_strength;
    a.gn = (float)(1.0 - guidance_strength);
    a.a = (float)(1.0 - sigma_min);
    a.cc = (float)(sigma_min + (1.0 - sigma_min) * t);
    a.dt = (float)(t - t_prev);
    a.gr = (float)guidance_rescale;
    a.one_m_gr = 1.0f - a.gr;
    // vector path: 16-byte aligned tensors and block bounds on whole vectors
    const int64_t ve = dtype == T2H_F32 ? 4 : 8;
    const bool al = T2H_EULER_VEC && aligned(a.x, 16) && aligned(a.v_pos, 16) && (a.mode == 0 || aligned(a.v_neg, 16)) &&
                    aligned(x_prev, 16) && aligned(pred_x0, 16);
    int64_t cover_lo = 0, cover_hi = n;
    if (a.mode == 2) {
        bool bounds_al = true;
        int64_t blocks = 0, stats = 0;
        if (n_seg_offsets > 0) {
            if (seg_offsets_host == nullptr) return fail(T2H_EINVAL, "%s: NULL seg_offsets", fn);
            const int nseg = n_seg_offsets - 1;
            if (nseg > kEulerMaxSeg) return fail(T2H_EUNSUPPORTED, "%s: more than %d segments", fn, kEulerMaxSeg);
            for (int s = 0; s <= nseg; ++s) {
                const int64_t o = seg_offsets_host[s];
                if (o < 0 || o > rows || (s > 0 && o < seg_offsets_host[s - 1]))
                    return fail(T2H_EINVAL, "%s: seg_offsets must be ordered within [0, rows]", fn);
                a.bounds[s] = o * row_size;
                bounds_al = bounds_al && a.bounds[s] % ve == 0;
            }
            a.uniform = 0;
            a.nseg = nseg;
            for (int s = 0; s < nseg; ++s) {
                const int64_t m = a.bounds[s + 1] - a.bounds[s];
                a.blk_base[s] = blocks;
                a.pbase[s] = stats;
                blocks += (m + kEulerChunk - 1) / kEulerChunk;
                stats += stats_blocks(m);
            }
            a.blk_base[nseg] = blocks;
            a.pbase[nseg] = stats;
            cover_lo = a.bounds[0];
            cover_hi = a.bounds[nseg];
        } else {
            a.uniform = 1;
            if (rows > INT32_MAX) return fail(T2H_EUNSUPPORTED, "%s: too many rows", fn);
            a.nseg = (int32_t)rows;
            a.pper = (int32_t)stats_blocks(row_size);
            blocks = rows * ((row_size + kEulerChunk - 1) / kEulerChunk);
            stats = rows * a.pper;
            bounds_al = row_size % ve == 0;
        }
        const int64_t need = stats * 32;
        if (builtin) {
            if (stats > kEulerScratchPartials)
                return fail(T2H_EUNSUPPORTED, "%s: the rescale needs %lld statistics blocks; the built-in scratch "
                            "holds %d (use t2h_flow_euler_step with a workspace)", fn, (long long)stats,
                            kEulerScratchPartials);
            double* sp = nullptr;
            if (hipError_t e = euler_scratch(&sp); e != hipSuccess) return hip_status(e, fn);
            workspace = sp;
            workspace_bytes = (int64_t)kEulerScratchPartials * 32;
        }
        if (workspace == nullptr || workspace_bytes < need)
            return fail(T2H_EINVAL, "%s: rescale needs a %lld-byte workspace", fn, (long long)need);
        if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return fail(T2H_EINVAL, "%s: workspace alignment", fn);
        a.partial = static_cast<double*>(workspace);
        a.nblocks = blocks;
        a.nstats = stats;
        a.vec = al && bounds_al ? 1 : 0;
        // one segment on whole vectors with room for the barrier: the
        // launcher may take the one-launch form
        const bool one_seg = n_seg_offsets > 0 ? a.nseg == 1 : rows == 1;
        if (one_seg && a.vec && workspace_bytes >= kFuseBytes) {
            a.fuse = 1;
            a.fuse_lo = n_seg_offsets > 0 ? a.bounds[0] : 0;
            a.fuse_hi = n_seg_offsets > 0 ? a.bounds[1] : n;
            a.fuse_ws = workspace;
            a.fuse_polls = fuse_wait_polls();
        }
    } else {
        a.nblocks = (n + kEulerChunk - 1) / kEulerChunk;
        a.vec = al && n % ve == 0 ? 1 : 0;
    }
    return hip_status(launch_euler(a, cover_lo, cover_hi, static_cast<hipStream_t>(stream)), fn);
}

int32_t t2h_flow_euler_step(const void* x_t, const void* v_pos, const void* v_neg, void* x_prev, void* pred_x0,
                            int64_t rows, int64_t row_size, int32_t dtype, double t, double t_prev,
                            double sigma_min, double guidance_strength, double guidance_rescale,
                            const int64_t* seg_offsets_host, int32_t n_seg_offsets, void* workspace,
                            int64_t workspace_bytes, void* stream) {
    return euler_step(x_t, v_pos, v_neg, x_prev, pred_x0, rows, row_size, dtype, t, t_prev, sigma_min,
                      guidance_strength, guidance_rescale, seg_offsets_host, n_seg_offsets, workspace,
                      workspace_bytes, false, stream, "t2h_flow_euler_step");
}

int32_t t2h_flow_euler_step_noalloc(const void* x_t, const void* v_pos, const void* v_neg, void* x_prev,
                                    void* pred_x0, int64_t rows, int64_t row_size, int32_t dtype, double t,
                                    double t_prev, double sigma_min, double guidance_strength,
                                    double guidance_rescale, const int64_t* seg_offsets_host, int32_t n_seg_offsets,
                                    void* stream) {
    return euler_step(x_t, v_pos, v_neg, x_prev, pred_x0, rows, row_size, dtype, t, t_prev, sigma_min,
                      guidance_strength, guidance_rescale, seg_offsets_host, n_seg_offsets, nullptr, 0, true,
                      stream, "t2h_flow_euler_step_noalloc");
}

// Resident-block glue over one const buffer: the pair at `off` is
// consts[off : off+c], consts[off+c : off+2c] (gpu/block.mojo:255-289).
static constexpr float kBlockEps = 1e-6f;   // gpu/block.mojo:44

static int32_t check_pair(const float* consts, int64_t rows, int32_t c, int32_t off, const char* fn) {
    if (rows < 0 || c <= 0) return fail(T2H_EINVAL, "%s: bad shape [%lld, %d]", fn, (long long)rows, c);
    if (off < 0) return fail(T2H_EINVAL, "%s: negative const offset %d", fn, off);
    if (consts == nullptr) return fail(T2H_EINVAL, "%s: NULL consts", fn);
    return T2H_OK;
}

int32_t t2h_ln_mod_rows(const void* x, void* dst, const float* consts, int64_t rows, int32_t c, int32_t off,
                        int32_t mode, int32_t dtype, void* stream) {
    const char* fn = "t2h_ln_mod_rows";
    if (int32_t rc = check_pair(consts, rows, c, off, fn)) return rc;
    if (mode != T2H_LN_MODULATE && mode != T2H_LN_AFFINE) return fail(T2H_EINVAL, "%s: bad mode %d", fn, mode);
    const float* a = consts + off;
    return t2h_ln_modulate(x, dst, rows, c, dtype, kBlockEps, mode, a, a + c, 0, nullptr, 1, 0, stream);
}

int32_t t2h_gate_add_bias_rows(void* x, const void* h, const float* consts, int64_t rows, int32_t c, int32_t off,
                               int32_t use_gate, int32_t dtype, void* stream) {
    const char* fn = "t2h_gate_add_bias_rows";
    if (int32_t rc = check_pair(consts, rows, c, off, fn)) return rc;
    if (use_gate != 0 && use_gate != 1) return fail(T2H_EINVAL, "%s: use_gate must be 0 or 1", fn);
    if (rows > 0 && x == nullptr) return fail(T2H_EINVAL, "%s: NULL x", fn);
    const float* a = consts + off;
    return t2h_gate_residual(x, h, x, a, use_gate ? a + c : nullptr, 0, rows, c, dtype, nullptr, 1, 0, stream);
}

int32_t t2h_block_join_ln(void* x, const void* h, void* dst, const float* consts, int64_t rows, int32_t c,
                          int32_t join_off, int32_t use_gate, int32_t norm_off, int32_t mode, int32_t dtype,
                          void* stream) {
    const char* fn = "t2h_block_join_ln";
    if (int32_t rc = check_pair(consts, rows, c, join_off, fn)) return rc;
    if (norm_off < 0) return fail(T2H_EINVAL, "%s: negative const offset %d", fn, norm_off);
    if (use_gate != 0 && use_gate != 1) return fail(T2H_EINVAL, "%s: use_gate must be 0 or 1", fn);
    if (mode != T2H_LN_MODULATE && mode != T2H_LN_AFFINE) return fail(T2H_EINVAL, "%s: bad mode %d", fn, mode);
    if (rows > 0 && (dst == x || dst == h)) return fail(T2H_EINVAL, "%s: dst must not alias x or h", fn);
    const float* j = consts + join_off;
    const float* n = consts + norm_off;
    return t2h_gate_residual_ln_modulate(x, h, x, dst, j, use_gate ? j + c : nullptr, 0, kBlockEps, mode, n, n + c, 0,
                                         rows, c, dtype, nullptr, 1, 0, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// host-pointer convenience wrappers
// ---------------------------------------------------------------------------
namespace {

// Device copies of host buffers, freed on scope exit.
struct DevBufs {
    std::vector<void*> ptrs;
    hipError_t err = hipSuccess;
    ~DevBufs() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <typename T>
    T* up(const T* host, int64_t n) {
        if (host == nullptr || err != hipSuccess) return nullptr;
        void* d = nullptr;
        err = hipMalloc(&d, (size_t)(n > 0 ? n : 1) * sizeof(T));
        if (err != hipSuccess) return nullptr;
        ptrs.push_back(d);
        if (n > 0) err = hipMemcpy(d, host, (size_t)n * sizeof(T), hipMemcpyHostToDevice);
        return static_cast<T*>(d);
    }
    template <typename T>
    T* alloc(int64_t n) {
        if (err != hipSuccess) return nullptr;
        void* d = nullptr;
        err = hipMalloc(&d, (size_t)(n > 0 ? n : 1) * sizeof(T));
        if (err != hipSuccess) return nullptr;
        ptrs.push_back(d);
        return static_cast<T*>(d);
    }
    template <typename T>
    hipError_t down(T* host, const T* dev, int64_t n) {
        if (err != hipSuccess) return err;
        if (host == nullptr || n <= 0) return hipSuccess;
        return hipMemcpy(host, dev, (size_t)n * sizeof(T), hipMemcpyDeviceToHost);
    }
};

int32_t finish(int32_t rc, DevBufs& b, const char* fn) {
    if (rc != T2H_OK) return rc;
    if (b.err != hipSuccess) return hip_status(b.err, fn);
    return hip_status(hipDeviceSynchronize(), fn);
}

}  // namespace

extern "C" {

int32_t t2h_h_ln_modulate(const float* x_host, float* out_host, int64_t rows, int32_t cols, float eps, int32_t mode,
                          const float* p0_host, const float* p1_host, const int64_t* offsets_host, int32_t nbatch,
                          int64_t rows_per_batch) {
    const char* fn = "t2h_h_ln_modulate";
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    const int64_t nb = offsets_host ? nbatch : (rows_per_batch > 0 ? (rows + rows_per_batch - 1) / rows_per_batch : 1);
    const int64_t np = mode == T2H_LN_MODULATE ? nb * cols : cols;
    DevBufs b;
    const float* x = b.up(x_host, rows * cols);
    float* out = b.alloc<float>(rows * cols);
    const float* p0 = b.up(p0_host, np);
    const float* p1 = b.up(p1_host, np);
    const int64_t* off = b.up(offsets_host, offsets_host ? nbatch + 1 : 0);
    if (b.err != hipSuccess) return hip_status(b.err, fn);
    int32_t rc = t2h_ln_modulate(x, out, rows, cols, T2H_F32, eps, mode, p0, p1, 0, off, nbatch, rows_per_batch, nullptr);
    rc = finish(rc, b, fn);
    if (rc == T2H_OK) rc = hip_status(b.down(out_host, out, rows * cols), fn);
    return rc;
}

int32_t t2h_h_qk_rmsnorm_rope(const float* q_host, const float* k_host, float* q_out_host, float* k_out_host,
                              int64_t rows, int32_t heads, int32_t head_dim, const float* gamma_q_host,
                              const float* gamma_k_host, int32_t use_rope, const float* freqs_host, int32_t freq_dim,
                              int32_t pos_dim, const float* phases_host, int64_t phase_rows,
                              const int32_t* coords_host, int32_t coord_cols, int32_t grid_res) {
    const char* fn = "t2h_h_qk_rmsnorm_rope";
    if (rows < 0 || heads <= 0 || head_dim <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    const int64_t n = rows * heads * head_dim;
    DevBufs b;
    const float* q = b.up(q_host, n);
    const float* k = b.up(k_host, n);
    float* qo = q_host ? b.alloc<float>(n) : nullptr;
    float* ko = k_host ? b.alloc<float>(n) : nullptr;
    const float* gq = b.up(gamma_q_host, (int64_t)heads * head_dim);
    const float* gk = b.up(gamma_k_host, (int64_t)heads * head_dim);
    const float* ph = b.up(phases_host, phase_rows * head_dim);
    const int32_t* co = b.up(coords_host, rows * coord_cols);
    if (b.err != hipSuccess) return hip_status(b.err, fn);
    int32_t rc = t2h_qk_rmsnorm_rope(q, k, qo, ko, rows, 0, 0, heads, head_dim, T2H_F32, nullptr, nullptr, gq, gk,
                                     use_rope, freqs_host, freq_dim, pos_dim, ph, phase_rows, co, coord_cols, grid_res,
                                     nullptr);
    rc = finish(rc, b, fn);
    if (rc == T2H_OK && q_out_host) rc = hip_status(b.down(q_out_host, qo, n), fn);
    if (rc == T2H_OK && k_out_host) rc = hip_status(b.down(k_out_host, ko, n), fn);
    return rc;
}

int32_t t2h_h_activation(const float* x_host, float* out_host, const float* bias_host, int64_t rows, int32_t cols,
                         int32_t kind) {
    const char* fn = "t2h_h_activation";
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    DevBufs b;
    const float* x = b.up(x_host, rows * cols);
    float* out = b.alloc<float>(rows * cols);
    const float* bias = b.up(bias_host, cols);
    if (b.err != hipSuccess) return hip_status(b.err, fn);
    int32_t rc = t2h_activation(x, out, bias, rows, cols, T2H_F32, kind, nullptr);
    rc = finish(rc, b, fn);
    if (rc == T2H_OK) rc = hip_status(b.down(out_host, out, rows * cols), fn);
    return rc;
}

int32_t t2h_h_gate_residual(const float* x_host, const float* h_host, float* out_host, const float* bias_host,
                            const float* gate_host, int64_t rows, int32_t cols, const int64_t* offsets_host,
                            int32_t nbatch, int64_t rows_per_batch) {
    const char* fn = "t2h_h_gate_residual";
    if (rows < 0 || cols <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    const int64_t nb = offsets_host ? nbatch : (rows_per_batch > 0 ? (rows + rows_per_batch - 1) / rows_per_batch : 1);
    DevBufs b;
    const float* x = b.up(x_host, rows * cols);
    const float* h = b.up(h_host, rows * cols);
    float* out = b.alloc<float>(rows * cols);
    const float* bias = b.up(bias_host, cols);
    const float* gate = b.up(gate_host, nb * cols);
    const int64_t* off = b.up(offsets_host, offsets_host ? nbatch + 1 : 0);
    if (b.err != hipSuccess) return hip_status(b.err, fn);
    int32_t rc = t2h_gate_residual(x, h, out, bias, gate, 0, rows, cols, T2H_F32, off, nbatch, rows_per_batch, nullptr);
    rc = finish(rc, b, fn);
    if (rc == T2H_OK) rc = hip_status(b.down(out_host, out, rows * cols), fn);
    return rc;
}

int32_t t2h_h_timestep_embedding(const float* t_host, float* out_host, int64_t n, int32_t dim, double max_period) {
    const char* fn = "t2h_h_timestep_embedding";
    if (n < 0 || dim <= 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    DevBufs b;
    const float* t = b.up(t_host, n);
    float* out = b.alloc<float>(n * dim);
    if (b.err != hipSuccess) return hip_status(b.err, fn);
    int32_t rc = t2h_timestep_embedding(t, out, n, dim, T2H_F32, max_period, nullptr);
    rc = finish(rc, b, fn);
    if (rc == T2H_OK) rc = hip_status(b.down(out_host, out, n * dim), fn);
    return rc;
}

int32_t t2h_h_coords_to_offsets(const int32_t* coords_host, int64_t rows, int32_t coord_cols, int32_t nbatch,
                                int64_t* offsets_host) {
    const char* fn = "t2h_h_coords_to_offsets";
    if (rows < 0 || coord_cols < 1 || nbatch < 0) return fail(T2H_EINVAL, "%s: bad shape", fn);
    DevBufs b;
    const int32_t* co = b.up(coords_host, rows * coord_cols);
    int64_t* off = b.alloc<int64_t>(nbatch + 1);
    int64_t* bad = b.alloc<int64_t>(1);
    if (b.err != hipSuccess) return hip_status(b.err, fn);
    int32_t rc = t2h_coords_to_offsets(co, rows, coord_cols, nbatch, off, bad, nullptr);
    rc = finish(rc, b, fn);
    if (rc != T2H_OK) return rc;
    int64_t first_bad = 0;
    rc = hip_status(b.down(&first_bad, bad, 1), fn);
    if (rc != T2H_OK) return rc;
    if (first_bad != INT64_MAX) {
        if (first_bad & 1) return fail(T2H_EBATCH_RANGE, "SparseTensor: batch index out of range");
        return fail(T2H_EBATCH_ORDER, "SparseTensor: batches must be ordered/contiguous");
    }
    return hip_status(b.down(offsets_host, off, nbatch + 1), fn);
}

}  // extern "C"
