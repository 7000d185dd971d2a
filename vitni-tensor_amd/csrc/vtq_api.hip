// vtq_api.hip -- the C ABI of libvtq (declared in include/vtq.h).
//
// Validation mirrors the reference's checks and messages per dtype arm
// (src/ops/quant.rs, src/model/forward_quantized.rs:663-785); where the
// reference would panic on a short slice this returns VTQ_E_INTERNAL.
// Compute always runs on the GPU: there is no CPU path in this library.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/vtq.h"
#include "vtq_kernels.h"

namespace {

struct DevBuf {
    void* ptr = nullptr;
    size_t cap = 0;
};

struct CachedWeight {
    size_t len = 0;
    void* dptr = nullptr;
};

}  // namespace

// The GEMM workspace of vtq_linear_device_noalloc: one fixed array per GPU
// (each device that loads the library holds its own copy until the process
// ends).  Host code never passes `scratch` itself to a kernel: its address
// on each device comes from hipGetSymbolAddress (vtq_create).
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct vtq_ctx {
    int device = 0;
    int num_cus = 0;
    hipStream_t stream = nullptr;
    DevBuf dx, dy;          // device staging for the host-pointer path
    DevBuf ws;              // kernel workspace (quantized activations of the GEMM path)
    void* scratch_ptr = nullptr;  // this device's `scratch` (vtq_linear_device_noalloc)
    void* hx = nullptr;     // pinned staging
    size_t hx_cap = 0;
    void* hy = nullptr;
    size_t hy_cap = 0;
    std::unordered_map<uintptr_t, CachedWeight> weights;
    std::string err;
};

namespace {

constexpr size_t kQ4K = 144, kQ6K = 210, kQ8_0 = 34, kQ5_0 = 22, kQ4_0 = 18;

int set_err(vtq_ctx* c, int code, const char* msg) {
    if (c) c->err = msg ? msg : "";
    return code;
}

int hip_fail(vtq_ctx* c, hipError_t e, const char* where) {
    std::string m = std::string("GpuError: ") + where + ": " + hipGetErrorString(e);
    if (c) c->err = m;
    return VTQ_E_GPU;
}

bool mul_ok(size_t a, size_t b, size_t* r) { return !__builtin_mul_overflow(a, b, r); }

int grow_dev(vtq_ctx* c, DevBuf& b, size_t bytes) {
    if (b.cap >= bytes) return VTQ_OK;
    if (b.ptr) (void)hipFree(b.ptr);
    b.ptr = nullptr;
    b.cap = 0;
    hipError_t e = hipMalloc(&b.ptr, bytes ? bytes : 16);
    if (e != hipSuccess) return hip_fail(c, e, "hipMalloc");
    b.cap = bytes;
    return VTQ_OK;
}

int grow_host(vtq_ctx* c, void*& p, size_t& cap, size_t bytes) {
    if (cap >= bytes) return VTQ_OK;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    cap = 0;
    hipError_t e = hipHostMalloc(&p, bytes ? bytes : 16, hipHostMallocDefault);
    if (e != hipSuccess) return hip_fail(c, e, "hipHostMalloc");
    cap = bytes;
    return VTQ_OK;
}

// Shape of one dtype arm after validation.
struct Plan {
    enum Kind { kQ4KInt, kQ4KGemm, kQ6KInt, kCanon } kind = kCanon;
    vtq::CanonFormat fmt = vtq::kCanonQ8_0;
    size_t row_bytes = 0;
    size_t w_need = 0;  // bytes of w the kernels read
};

// Validate one linear_dispatch arm.  `serial_names` selects the messages of
// the serial k-quant functions; otherwise those of the row-parallel twins,
// which the reference's dispatch uses for out_feat >= 512 (PAR_MIN_ROWS,
// src/model/forward_quantized.rs:710, :734).
int plan_linear(vtq_ctx* c, int type, int regime, size_t w_len, size_t batch, size_t in_feat,
                size_t out_feat, bool serial_names, Plan* p) {
    if (batch > (size_t)INT_MAX || in_feat > (size_t)INT_MAX || out_feat > (size_t)INT_MAX)
        return set_err(c, VTQ_E_NOT_IMPLEMENTED, "vtq: dimension exceeds INT_MAX");
    size_t need = 0;
    switch (type) {
    case VTQ_TYPE_Q4_K:
        if (regime == VTQ_REGIME_FLOAT_FUSED) {
            if (in_feat % 256 != 0)
                return set_err(c, VTQ_E_INTERNAL, "linear_q4_k_fused: in_feat not a multiple of 256");
            p->row_bytes = (in_feat / 256) * kQ4K;
            if (!mul_ok(out_feat, p->row_bytes, &need) || w_len < need)
                return set_err(c, VTQ_E_INTERNAL, "linear_q4_k_fused: weight shape mismatch");
            p->kind = Plan::kCanon;
            p->fmt = vtq::kCanonQ4KFloat;
        } else if (regime == VTQ_REGIME_INTEGER) {
            if (in_feat % 256 != 0)
                return set_err(c, VTQ_E_INTERNAL, serial_names ? "linear_q4_k_integer: in_feat not a multiple of 256"
                                                               : "linear_q4_k_integer_parallel: in_feat % 256");
            p->row_bytes = (in_feat / 256) * kQ4K;
            if (!mul_ok(out_feat, p->row_bytes, &need) || w_len < need)
                return set_err(c, VTQ_E_INTERNAL, serial_names ? "linear_q4_k_integer: weight shape mismatch"
                                                               : "linear_q4_k_integer_parallel: weight shape");
            p->kind = (batch >= (size_t)vtq::kGemmMinBatch && in_feat <= (size_t)vtq::q4k_gemm_max_in_feat())
                          ? Plan::kQ4KGemm
                          : Plan::kQ4KInt;
        } else {
            return set_err(c, VTQ_E_INVALID_ARGUMENT, "vtq: unknown regime");
        }
        break;
    case VTQ_TYPE_Q6_K:
        if (in_feat % 256 != 0)
            return set_err(c, VTQ_E_INTERNAL, serial_names ? "linear_q6_k_integer: in_feat not a multiple of 256"
                                                           : "linear_q6_k_integer_parallel: in_feat % 256");
        p->row_bytes = (in_feat / 256) * kQ6K;
        if (!mul_ok(out_feat, p->row_bytes, &need) || w_len < need)
            return set_err(c, VTQ_E_INTERNAL, serial_names ? "linear_q6_k_integer: weight shape mismatch"
                                                           : "linear_q6_k_integer_parallel: weight shape");
        p->kind = Plan::kQ6KInt;
        break;
    case VTQ_TYPE_Q8_0:
    case VTQ_TYPE_Q5_0: {
        const bool q8 = type == VTQ_TYPE_Q8_0;
        if (in_feat % 32 != 0)
            return set_err(c, VTQ_E_INTERNAL, q8 ? "Q8_0: in_feat must be a multiple of 32"
                                                 : "Q5_0: in_feat must be a multiple of 32");
        p->row_bytes = (in_feat / 32) * (q8 ? kQ8_0 : kQ5_0);
        if (!mul_ok(out_feat, p->row_bytes, &need) || w_len < need)
            return set_err(c, VTQ_E_INTERNAL, q8 ? "linear_dispatch Q8_0: weight blob too small"
                                                 : "linear_dispatch Q5_0: weight blob too small");
        p->kind = Plan::kCanon;
        p->fmt = q8 ? vtq::kCanonQ8_0 : vtq::kCanonQ5_0;
        break;
    }
    case VTQ_TYPE_Q4_0:
        if (in_feat % 32 != 0) return set_err(c, VTQ_E_INTERNAL, "linear_q4_0: in_feat must be multiple of 32");
        p->row_bytes = (in_feat / 32) * kQ4_0;
        if (!mul_ok(out_feat, p->row_bytes, &need) || w_len != need)
            return set_err(c, VTQ_E_INTERNAL, "linear_q4_0: weight blob length mismatch");
        p->kind = Plan::kCanon;
        p->fmt = vtq::kCanonQ4_0;
        break;
    case VTQ_TYPE_F32:
        if (!mul_ok(in_feat, 4, &p->row_bytes) || !mul_ok(out_feat, p->row_bytes, &need) || w_len != need)
            return set_err(c, VTQ_E_INTERNAL, "linear_dispatch F32: weight size mismatch");
        p->kind = Plan::kCanon;
        p->fmt = vtq::kCanonF32;
        break;
    default:
        return set_err(c, VTQ_E_NOT_IMPLEMENTED,
                       "forward_quantized::linear_dispatch: weight dtype not Q4_0 / Q4_K / Q5_0 / Q6_K / Q8_0 / F32");
    }
    p->w_need = need;
    return VTQ_OK;
}

// Rows longer than the kernels hold run as aligned segments (see
// vtq_kernels.h): the segment length in inputs, or 0 when the plan needs none.
size_t segment_inputs(const Plan& p, size_t in_feat) {
    if ((p.kind == Plan::kQ4KInt || p.kind == Plan::kQ6KInt) && in_feat > (size_t)vtq::kquant_max_in_feat())
        return (size_t)vtq::kquant_max_in_feat();
    if (p.kind == Plan::kCanon && in_feat > (size_t)vtq::canon_max_in_feat()) return (size_t)vtq::canon_max_in_feat();
    return 0;
}

// Batch rows per pass of a segmented plan and the workspace that pass needs:
// the segments' y slices, plus (canonical dot, batch > 1) one segment of x
// gathered into contiguous rows.  Passes are sized to stay under `cap`
// bytes where one batch row fits; 0 rows if not even one does.
size_t segment_rows(const Plan& p, size_t batch, size_t in_feat, size_t out_feat, size_t cap, size_t* ws_bytes) {
    const size_t seg = segment_inputs(p, in_feat), nseg = (in_feat + seg - 1) / seg;
    const bool gather = p.kind == Plan::kCanon;
    auto need = [&](size_t rows) {
        return (nseg * rows * out_feat + (gather && rows > 1 ? rows * seg : 0)) * 4 + 256;
    };
    size_t rows = batch < 65535 ? batch : 65535;
    while (rows > 1 && need(rows) > cap) rows = (rows + 1) / 2;
    *ws_bytes = need(rows);
    return need(rows) <= cap ? rows : 0;
}

int run_segmented(vtq_ctx* c, const Plan& p, const float* dx, const uint8_t* dw, float* dy, size_t batch,
                  size_t in_feat, size_t out_feat, hipStream_t s, void* fixed_ws, size_t fixed_ws_bytes) {
    const size_t seg = segment_inputs(p, in_feat), nseg = (in_feat + seg - 1) / seg;
    size_t ws_bytes = 0;
    const size_t rows = segment_rows(p, batch, in_feat, out_feat, fixed_ws ? fixed_ws_bytes : ((size_t)256 << 20),
                                     &ws_bytes);
    if (rows == 0)
        return set_err(c, VTQ_E_NOT_IMPLEMENTED, "vtq: the segment workspace of one batch row exceeds the scratch");
    void* ws = fixed_ws;
    if (!ws) {
        if (int rc = grow_dev(c, c->ws, ws_bytes)) return rc;
        ws = c->ws.ptr;
    }
    float* part = static_cast<float*>(ws);
    hipError_t e = hipSuccess;
    for (size_t b0 = 0; b0 < batch; b0 += rows) {
        const int nb = (int)(batch - b0 < rows ? batch - b0 : rows);
        float* xg = part + nseg * (size_t)nb * out_feat;
        for (size_t k = 0; k < nseg; k++) {
            const size_t i0 = k * seg;
            const int len = (int)(in_feat - i0 < seg ? in_feat - i0 : seg);
            float* yk = part + k * (size_t)nb * out_feat;
            if (p.kind == Plan::kCanon) {
                // byte offset of input i0 in a row: i0 is a multiple of every block size
                const size_t off = p.fmt == vtq::kCanonF32 ? i0 * 4
                                   : p.fmt == vtq::kCanonQ8_0 ? i0 / 32 * kQ8_0
                                   : p.fmt == vtq::kCanonQ5_0 ? i0 / 32 * kQ5_0
                                   : p.fmt == vtq::kCanonQ4_0 ? i0 / 32 * kQ4_0
                                                               : i0 / 256 * kQ4K;
                const float* xs = dx + b0 * in_feat + i0;
                if (nb > 1) {
                    e = vtq::launch_gather_cols(dx + b0 * in_feat, in_feat, i0, len, nb, xg, s);
                    if (e != hipSuccess) return hip_fail(c, e, "kernel launch");
                    xs = xg;
                }
                e = vtq::launch_canon_segment(p.fmt, xs, dw + off, p.row_bytes, p.w_need - off, yk, nb, len,
                                              (int)out_feat, s);
            } else {
                const size_t off = i0 / 256 * (p.kind == Plan::kQ4KInt ? kQ4K : kQ6K);
                e = vtq::launch_kquant_segment(p.kind == Plan::kQ4KInt ? 12 : 14, dx + b0 * in_feat + i0, (int)in_feat,
                                               dw + off, p.row_bytes, yk, nb, len, (int)out_feat, c->num_cus, s);
            }
            if (e != hipSuccess) return hip_fail(c, e, "kernel launch");
        }
        e = vtq::launch_segment_tree(part, (size_t)nb * out_feat, (int)nseg, dy + b0 * out_feat, s);
        if (e != hipSuccess) return hip_fail(c, e, "kernel launch");
    }
    return VTQ_OK;
}

// Enqueue the kernels of a validated plan.  `fixed_ws` (when not null) is a
// caller-provided workspace of `fixed_ws_bytes` (the GEMM's size already
// checked); else the context's workspace grows on demand.
int run_plan(vtq_ctx* c, const Plan& p, const float* dx, const uint8_t* dw, float* dy, size_t batch,
             size_t in_feat, size_t out_feat, hipStream_t s, void* fixed_ws = nullptr, size_t fixed_ws_bytes = 0) {
    if (batch == 0 || out_feat == 0) return VTQ_OK;
    hipError_t e = hipSuccess;
    if (in_feat == 0) {  // every reduction is over nothing: fixed_tree([]) == 0.0
        e = vtq::launch_fill(dy, batch * out_feat, 0.0f, s);
        return e == hipSuccess ? VTQ_OK : hip_fail(c, e, "fill");
    }
    if (segment_inputs(p, in_feat)) return run_segmented(c, p, dx, dw, dy, batch, in_feat, out_feat, s, fixed_ws,
                                                         fixed_ws_bytes);
    if (p.kind == Plan::kQ4KGemm) {
        // the launcher walks the batch in chunks that fit the workspace
        void* ws = fixed_ws;
        if (!ws) {
            int rc = grow_dev(c, c->ws, vtq::q4k_gemm_workspace_bytes((int)batch, (int)in_feat));
            if (rc) return rc;
            ws = c->ws.ptr;
        }
        e = vtq::launch_q4k_gemm(dx, dw, dy, (int)batch, (int)in_feat, (int)out_feat, ws, s);
        return e == hipSuccess ? VTQ_OK : hip_fail(c, e, "kernel launch");
    }
    const size_t kMaxGridY = 65535;
    for (size_t b0 = 0; b0 < batch; b0 += kMaxGridY) {
        const int nb = (int)(batch - b0 < kMaxGridY ? batch - b0 : kMaxGridY);
        const float* xb = dx + b0 * in_feat;
        float* yb = dy + b0 * out_feat;
        switch (p.kind) {
        case Plan::kQ4KInt:
            e = vtq::launch_q4k_gemv(xb, dw, yb, nb, (int)in_feat, (int)out_feat, c->num_cus, s);
            break;
        case Plan::kQ4KGemm:
            break;
        case Plan::kQ6KInt:
            e = vtq::launch_q6k_gemv(xb, dw, yb, nb, (int)in_feat, (int)out_feat, c->num_cus, s);
            break;
        case Plan::kCanon:
            e = vtq::launch_canon_gemv(p.fmt, xb, dw, p.row_bytes, yb, nb, (int)in_feat, (int)out_feat, c->num_cus, s);
            break;
        }
        if (e != hipSuccess) return hip_fail(c, e, "kernel launch");
    }
    return VTQ_OK;
}

int cached_weight(vtq_ctx* c, const uint8_t* w, size_t w_len, const uint8_t** out) {
    auto it = c->weights.find(reinterpret_cast<uintptr_t>(w));
    if (it != c->weights.end() && it->second.len == w_len) {
        *out = static_cast<const uint8_t*>(it->second.dptr);
        return VTQ_OK;
    }
    if (it != c->weights.end()) {
        (void)hipFree(it->second.dptr);
        c->weights.erase(it);
    }
    void* d = nullptr;
    // rounded up to 16 bytes: the canonical-dot kernels fetch whole 16-byte chunks
    hipError_t e = hipMalloc(&d, (w_len + 15) / 16 * 16 + 16);
    if (e != hipSuccess) return hip_fail(c, e, "hipMalloc(weights)");
    if (w_len) {
        e = hipMemcpy(d, w, w_len, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return hip_fail(c, e, "hipMemcpy(weights)");
        }
    }
    c->weights[reinterpret_cast<uintptr_t>(w)] = CachedWeight{w_len, d};
    *out = static_cast<const uint8_t*>(d);
    return VTQ_OK;
}

int linear_host(vtq_ctx* c, int type, int regime, const float* x, size_t x_len, const uint8_t* w, size_t w_len,
                float* y, size_t y_len, size_t batch, size_t in_feat, size_t out_feat, bool serial_names) {
    if (!c) return VTQ_E_INVALID_ARGUMENT;
    c->err.clear();
    Plan p;
    int rc = plan_linear(c, type, regime, w_len, batch, in_feat, out_feat, serial_names, &p);
    if (rc) return rc;
    size_t nx = 0, ny = 0;
    if (!mul_ok(batch, in_feat, &nx) || !mul_ok(batch, out_feat, &ny))
        return set_err(c, VTQ_E_INTERNAL, "vtq: batch * features overflows");
    if (type == VTQ_TYPE_Q4_0) {  // linear_q4_0_cpu checks exact lengths (src/ops/quant.rs:1544-1549)
        if (x_len != nx) return set_err(c, VTQ_E_INTERNAL, "linear_q4_0: x size mismatch");
        if (y_len != ny) return set_err(c, VTQ_E_INTERNAL, "linear_q4_0: y_out size mismatch");
    }
    if (x_len < nx) return set_err(c, VTQ_E_INTERNAL, "vtq: x shorter than batch * in_feat");
    if (y_len < ny) return set_err(c, VTQ_E_INTERNAL, "vtq: y shorter than batch * out_feat");
    if ((nx && !x) || (ny && !y) || (p.w_need && !w)) return set_err(c, VTQ_E_INVALID_ARGUMENT, "vtq: null pointer");
    if (ny == 0) return VTQ_OK;
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return hip_fail(c, e, "hipSetDevice");
    const uint8_t* dw = nullptr;
    if ((rc = cached_weight(c, w, p.w_need, &dw))) return rc;
    if ((rc = grow_dev(c, c->dx, nx * 4 + 16))) return rc;
    if ((rc = grow_dev(c, c->dy, ny * 4 + 16))) return rc;
    if ((rc = grow_host(c, c->hx, c->hx_cap, nx * 4 + 16))) return rc;
    if ((rc = grow_host(c, c->hy, c->hy_cap, ny * 4 + 16))) return rc;
    if (nx) {
        std::memcpy(c->hx, x, nx * 4);
        e = hipMemcpyAsync(c->dx.ptr, c->hx, nx * 4, hipMemcpyHostToDevice, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "hipMemcpyAsync(x)");
    }
    rc = run_plan(c, p, static_cast<const float*>(c->dx.ptr), dw, static_cast<float*>(c->dy.ptr), batch, in_feat,
                  out_feat, c->stream);
    if (rc) return rc;
    e = hipMemcpyAsync(c->hy, c->dy.ptr, ny * 4, hipMemcpyDeviceToHost, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "hipMemcpyAsync(y)");
    e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "hipStreamSynchronize");
    std::memcpy(y, c->hy, ny * 4);
    return VTQ_OK;
}

}  // namespace

namespace vtq {

hipError_t allow_dynamic_lds(const void* kernel, size_t bytes) {
    if (bytes <= 65536) return hipSuccess;
    // (device, kernel) -> limit set; a fixed table (no heap: the no-alloc
    // entry point runs through here), set anew every launch once it is full
    struct Raised {
        int dev;
        const void* kernel;
        size_t bytes;
    };
    static std::mutex mu;
    static Raised raised[128];
    static int n_raised = 0;
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev)) return e;
    std::lock_guard<std::mutex> lock(mu);
    Raised* slot = nullptr;
    for (int i = 0; i < n_raised; i++)
        if (raised[i].dev == dev && raised[i].kernel == kernel) slot = &raised[i];
    if (slot && slot->bytes >= bytes) return hipSuccess;
    if (hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes)) return e;
    if (!slot && n_raised < 128) slot = &raised[n_raised++];
    if (slot) *slot = Raised{dev, kernel, bytes};
    return hipSuccess;
}

}  // namespace vtq

extern "C" {

const char* vtq_version(void) { return "vtq 0.3.0 (gfx950)"; }

int vtq_create(int device, vtq_ctx** out) {
    if (!out) return VTQ_E_INVALID_ARGUMENT;
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || device < 0 || device >= n) return VTQ_E_GPU;
    e = hipSetDevice(device);
    if (e != hipSuccess) return VTQ_E_GPU;
    vtq_ctx* c = new (std::nothrow) vtq_ctx();
    if (!c) return VTQ_E_GPU;
    c->device = device;
    if (hipDeviceGetAttribute(&c->num_cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        c->num_cus <= 0)
        c->num_cus = 256;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return VTQ_E_GPU;
    }
    // this device's copy of `scratch` (the device is current)
    if (hipGetSymbolAddress(&c->scratch_ptr, HIP_SYMBOL(scratch)) != hipSuccess || !c->scratch_ptr) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return VTQ_E_GPU;
    }
    *out = c;
    return VTQ_OK;
}

void vtq_destroy(vtq_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (auto& kv : c->weights) (void)hipFree(kv.second.dptr);
    if (c->dx.ptr) (void)hipFree(c->dx.ptr);
    if (c->dy.ptr) (void)hipFree(c->dy.ptr);
    if (c->ws.ptr) (void)hipFree(c->ws.ptr);
    if (c->hx) (void)hipHostFree(c->hx);
    if (c->hy) (void)hipHostFree(c->hy);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

const char* vtq_last_error(const vtq_ctx* c) { return c ? c->err.c_str() : "vtq: null context"; }

// The reference's dispatch names the row-parallel k-quant functions in its
// errors only in the std-parallel build and for out_feat >= PAR_MIN_ROWS
// (forward_quantized.rs:704-750); the default build always calls the serial
// ones.
static bool dispatch_serial_names(int regime, size_t out_feat) {
    return regime == VTQ_REGIME_FLOAT_FUSED || out_feat < 512;
}

int vtq_linear(vtq_ctx* c, int type, int regime, const float* x, size_t x_len, const uint8_t* w, size_t w_len,
               float* y, size_t y_len, size_t batch, size_t in_feat, size_t out_feat) {
    return linear_host(c, type, regime, x, x_len, w, w_len, y, y_len, batch, in_feat, out_feat,
                       dispatch_serial_names(regime, out_feat));
}

int vtq_linear_q4_k_integer(vtq_ctx* c, const float* x, size_t x_len, const uint8_t* w, size_t w_len, float* y,
                            size_t y_len, size_t batch, size_t in_feat, size_t out_feat) {
    return linear_host(c, VTQ_TYPE_Q4_K, VTQ_REGIME_INTEGER, x, x_len, w, w_len, y, y_len, batch, in_feat, out_feat,
                       true);
}

int vtq_linear_q6_k_integer(vtq_ctx* c, const float* x, size_t x_len, const uint8_t* w, size_t w_len, float* y,
                            size_t y_len, size_t batch, size_t in_feat, size_t out_feat) {
    return linear_host(c, VTQ_TYPE_Q6_K, VTQ_REGIME_INTEGER, x, x_len, w, w_len, y, y_len, batch, in_feat, out_feat,
                       true);
}

int vtq_linear_q4_k_fused(vtq_ctx* c, const float* x, size_t x_len, const uint8_t* w, size_t w_len, float* y,
                          size_t y_len, size_t batch, size_t in_feat, size_t out_feat) {
    return linear_host(c, VTQ_TYPE_Q4_K, VTQ_REGIME_FLOAT_FUSED, x, x_len, w, w_len, y, y_len, batch, in_feat,
                       out_feat, true);
}

int vtq_linear_q4_0(vtq_ctx* c, const float* x, size_t x_len, const uint8_t* w, size_t w_len, float* y,
                    size_t y_len, size_t batch, size_t in_feat, size_t out_feat) {
    return linear_host(c, VTQ_TYPE_Q4_0, VTQ_REGIME_INTEGER, x, x_len, w, w_len, y, y_len, batch, in_feat, out_feat,
                       true);
}

int vtq_release_weights(vtq_ctx* c, const uint8_t* w) {
    if (!c) return VTQ_E_INVALID_ARGUMENT;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    if (!w) {
        for (auto& kv : c->weights) (void)hipFree(kv.second.dptr);
        c->weights.clear();
        return VTQ_OK;
    }
    auto it = c->weights.find(reinterpret_cast<uintptr_t>(w));
    if (it != c->weights.end()) {
        (void)hipFree(it->second.dptr);
        c->weights.erase(it);
    }
    return VTQ_OK;
}

int vtq_linear_device(vtq_ctx* c, int type, int regime, const float* d_x, const uint8_t* d_w, size_t w_len,
                      float* d_y, size_t batch, size_t in_feat, size_t out_feat, void* stream) {
    if (!c) return VTQ_E_INVALID_ARGUMENT;
    c->err.clear();
    Plan p;
    int rc = plan_linear(c, type, regime, w_len, batch, in_feat, out_feat, dispatch_serial_names(regime, out_feat), &p);
    if (rc) return rc;
    size_t nx = 0, ny = 0;
    if (!mul_ok(batch, in_feat, &nx) || !mul_ok(batch, out_feat, &ny))
        return set_err(c, VTQ_E_INTERNAL, "vtq: batch * features overflows");
    if ((nx && !d_x) || (ny && !d_y) || (p.w_need && !d_w)) return set_err(c, VTQ_E_INVALID_ARGUMENT, "vtq: null pointer");
    if ((reinterpret_cast<uintptr_t>(d_x) & 15u) || (reinterpret_cast<uintptr_t>(d_w) & 15u))
        return set_err(c, VTQ_E_INVALID_ARGUMENT, "vtq: device x and w must be 16-byte aligned");
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return hip_fail(c, e, "hipSetDevice");
    return run_plan(c, p, d_x, d_w, d_y, batch, in_feat, out_feat, static_cast<hipStream_t>(stream));
}

int vtq_linear_device_noalloc(vtq_ctx* c, int type, int regime, const float* d_x, const uint8_t* d_w, size_t w_len,
                              float* d_y, size_t batch, size_t in_feat, size_t out_feat, void* stream) {
    if (!c) return VTQ_E_INVALID_ARGUMENT;
    c->err.clear();
    Plan p;
    int rc = plan_linear(c, type, regime, w_len, batch, in_feat, out_feat, dispatch_serial_names(regime, out_feat), &p);
    if (rc) return rc;
    size_t nx = 0, ny = 0;
    if (!mul_ok(batch, in_feat, &nx) || !mul_ok(batch, out_feat, &ny))
        return set_err(c, VTQ_E_INTERNAL, "vtq: batch * features overflows");
    if ((nx && !d_x) || (ny && !d_y) || (p.w_need && !d_w)) return set_err(c, VTQ_E_INVALID_ARGUMENT, "vtq: null pointer");
    if ((reinterpret_cast<uintptr_t>(d_x) & 15u) || (reinterpret_cast<uintptr_t>(d_w) & 15u))
        return set_err(c, VTQ_E_INVALID_ARGUMENT, "vtq: device x and w must be 16-byte aligned");
    if (p.kind == Plan::kQ4KGemm && vtq::q4k_gemm_workspace_bytes((int)batch, (int)in_feat) > kScratchBytes)
        return set_err(c, VTQ_E_NOT_IMPLEMENTED,
                       "vtq_linear_device_noalloc: the GEMM workspace of batch x in_feat exceeds the 32 MiB scratch");
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return hip_fail(c, e, "hipSetDevice");
    return run_plan(c, p, d_x, d_w, d_y, batch, in_feat, out_feat, static_cast<hipStream_t>(stream), c->scratch_ptr,
                    kScratchBytes);
}

}  // extern "C"
