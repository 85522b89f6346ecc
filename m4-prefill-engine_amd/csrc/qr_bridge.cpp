// qr_bridge.cpp -- the C-ABI (include/m4_mlx_bridge.h) over the HIP kernels.
//
// Mirrors core/bridge/m4_mlx_bridge.mm:79-343: same entry points, same
// validation order and error codes, asynchronous dispatch + synchronize.
// Where the reference wraps unified host memory zero-copy (:38-55), this
// bridge takes device pointers directly and stages anything else (pageable
// host memory, or device buffers too misaligned for 16-byte vector loads)
// through bridge-owned device memory.
#include <hip/hip_runtime.h>

#include <sys/uio.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/m4_mlx_bridge.h"
#include "qr_formats.h"
#include "qr_host.h"
#include "qr_kernels.h"
#include "qr_registry.h"

namespace {

using qr::has_kernels;
using qr::host_range_ok;
using qr::is_projection_format;
using qr::validate;

std::mutex g_mu;
bool g_initialized = false;
int g_device = 0;
hipStream_t g_own_stream = nullptr;
hipStream_t g_stream = nullptr;
thread_local std::string g_last_error;  // per thread, like errno: a caller reads the message of its own failed call

struct Staged {
    void* dev;
    void* host;      // non-null: copy dev -> host at synchronize (once armed)
    size_t bytes;
    bool armed;      // set once the dispatch that staged it has launched its kernels
    size_t cap;      // bytes of the staging allocation (>= bytes)
};
std::vector<Staged> g_staged;      // returned to the staging pool at synchronize
size_t g_staged_bytes = 0;

// Staging allocations are reused: synchronize returns them to this free list
// and the next staged buffer takes the smallest one that fits, so a caller
// that passes host (or misaligned) buffers on every call allocates only while
// its working set grows.  The list keeps at most kPoolMaxBytes; beyond that
// the largest free allocations are released.
std::vector<std::pair<void*, size_t>> g_pool;
size_t g_pool_bytes = 0;
constexpr size_t kPoolMaxBytes = size_t(4) << 30;

hipError_t pool_take(size_t bytes, void** out, size_t* cap) {
    int best = -1;
    for (int i = 0; i < (int)g_pool.size(); i++)
        if (g_pool[i].second >= bytes && (best < 0 || g_pool[i].second < g_pool[best].second)) best = i;
    if (best >= 0) {
        *out = g_pool[best].first;
        *cap = g_pool[best].second;
        g_pool_bytes -= *cap;
        g_pool.erase(g_pool.begin() + best);
        return hipSuccess;
    }
    // whole MiB above 1 MiB, powers of two below: sizes that later calls reuse
    size_t c = 256;
    if (bytes > (size_t(1) << 20)) c = (bytes + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    else
        while (c < bytes) c <<= 1;
    *cap = c;
    return hipMalloc(out, c);
}

void pool_give(void* p, size_t cap) {
    g_pool.emplace_back(p, cap);
    g_pool_bytes += cap;
    while (g_pool_bytes > kPoolMaxBytes) {
        size_t big = 0;
        for (size_t i = 1; i < g_pool.size(); i++)
            if (g_pool[i].second > g_pool[big].second) big = i;
        (void)hipFree(g_pool[big].first);
        g_pool_bytes -= g_pool[big].second;
        g_pool.erase(g_pool.begin() + big);
    }
}

// Grow-only scratch for the layer composition, and for the dequantized fp16
// K / V^T cache of the standalone attention entry points.
void* g_ws = nullptr;
size_t g_ws_bytes = 0;
void* g_attn_ws = nullptr;
size_t g_attn_ws_bytes = 0;
// Workspaces outgrown by a larger call.  A HIP graph captured earlier may
// still hold their addresses, so they stay allocated until shutdown.
std::vector<void*> g_retired;
size_t g_retired_bytes = 0;

void set_error(const char* where, hipError_t e) {
    char buf[256];
    snprintf(buf, sizeof(buf), "%s: %s", where, hipGetErrorString(e));
    g_last_error = buf;
}

// Classify a pointer: device-accessible address or null if it must be staged.
void* device_view(void* p) {
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged ||
        attr.type == hipMemoryTypeUnified)
        return attr.devicePointer ? attr.devicePointer : p;
    if (attr.type == hipMemoryTypeHost && attr.devicePointer) return attr.devicePointer;
    return nullptr;
}

// Device pointer usable by the kernels for buffer `p`: the pointer itself if it
// is device memory aligned to `align`, else a staged copy.  For outputs
// (`out`), the staged copy is written back at synchronize.  Returns null on
// allocation/copy failure.
// Host outputs of earlier dispatches are copied back at synchronize.  A host
// input that overlaps one of them must see that result (the reference's
// in-order queue on zero-copy buffers does), so before such an input is
// staged the stream is drained and every pending host output written back,
// in dispatch order.
void flush_pending_host_outputs(const void* p, size_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p), b = a + bytes;
    bool overlap = false;
    for (const auto& st : g_staged) {
        if (!st.host || !st.armed) continue;
        const uintptr_t sa = reinterpret_cast<uintptr_t>(st.host), sb = sa + st.bytes;
        overlap |= sa < b && a < sb;
    }
    if (!overlap) return;
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) set_error("hipStreamSynchronize", e);
    for (auto& st : g_staged) {
        if (!st.host || !st.armed) continue;
        e = hipMemcpy(st.host, st.dev, st.bytes, hipMemcpyDeviceToHost);
        if (e != hipSuccess) set_error("hipMemcpy(stage out)", e);
        st.host = nullptr;
    }
}

void* resolve(void* p, size_t bytes, size_t align, bool in, bool out) {
    void* d = device_view(p);
    if (d && (reinterpret_cast<uintptr_t>(d) % align) == 0) return d;
    if (!d && !host_range_ok(p, bytes, out)) {
        g_last_error = "host buffer range is not accessible";
        return nullptr;
    }
    if (!d && in) flush_pending_host_outputs(p, bytes);
    void* s = nullptr;
    size_t cap = 0;
    hipError_t e = pool_take(bytes ? bytes : 16, &s, &cap);
    if (e != hipSuccess) {
        set_error("hipMalloc(staging)", e);
        return nullptr;
    }
    if (in) {
        e = d ? hipMemcpyAsync(s, d, bytes, hipMemcpyDeviceToDevice, g_stream)
              : hipMemcpyAsync(s, p, bytes, hipMemcpyHostToDevice, g_stream);
        if (e != hipSuccess) {
            set_error("hipMemcpyAsync(stage in)", e);
            pool_give(s, cap);
            return nullptr;
        }
    }
    // Device outputs that were only misaligned are copied back on the stream
    // right after the kernel (see finish_outputs); host outputs at synchronize.
    g_staged.push_back({s, out ? p : nullptr, bytes, false, cap});
    g_staged_bytes += bytes;
    return s;
}

// After the launches of one dispatch: device-resident outputs that were staged
// (misaligned) are copied back in stream order.
void finish_outputs() {
    for (auto& st : g_staged) {
        if (st.armed) continue;
        st.armed = true;  // a dispatch that fails before its launches never arms its outputs
        if (!st.host) continue;
        void* d = device_view(st.host);
        if (d) {
            (void)hipMemcpyAsync(d, st.dev, st.bytes, hipMemcpyDeviceToDevice, g_stream);
            st.host = nullptr;  // done
        }
    }
}

// A dispatch that fails -- buffers that could not all be staged (-5), or a
// launch error (-6) -- never copies its staged outputs back: the caller's
// output buffers are left untouched.
int dispatch_failed(int rc) {
    for (auto& st : g_staged)
        if (!st.armed) {
            st.armed = true;
            st.host = nullptr;
        }
    return rc;
}
int staging_failed() { return dispatch_failed(-5); }

// Ends a dispatch: outputs armed on success, disarmed on failure.
int finish(int rc) {
    if (rc) return dispatch_failed(rc);
    finish_outputs();
    return 0;
}

void sync_and_release() {
    if (!g_stream) return;
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) set_error("hipStreamSynchronize", e);
    for (auto& st : g_staged) {
        if (st.host && st.armed) {
            e = hipMemcpy(st.host, st.dev, st.bytes, hipMemcpyDeviceToHost);
            if (e != hipSuccess) set_error("hipMemcpy(stage out)", e);
        }
        pool_give(st.dev, st.cap);
    }
    g_staged.clear();
    g_staged_bytes = 0;
}



// Split-K workspace (fp32 partials) shared by the small-M and tiled kernels;
// launches are ordered on the bridge stream, grow-only.
float* g_sk_ws = nullptr;
size_t g_sk_ws_floats = 0;

// Makes `buf` hold at least `need` bytes.  Growing allocates a new buffer and
// retires the old one (kept until shutdown: a graph captured before may
// still launch kernels that use it).  Allocation is not allowed while the
// stream is being captured: the call must have run once at its size first.
hipError_t grow(void** buf, size_t* bytes, size_t need, bool zero, const char* what) {
    if (need <= *bytes) return hipSuccess;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g_stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        g_last_error = std::string(what) +
                       ": workspace must grow while the stream is being captured; run the call once at this size "
                       "before capturing it";
        return hipErrorStreamCaptureUnsupported;
    }
    void* nb = nullptr;
    hipError_t e = hipMalloc(&nb, need);
    if (e == hipSuccess && zero) e = hipMemset(nb, 0, need);
    if (e != hipSuccess) {
        if (nb) (void)hipFree(nb);
        set_error(what, e);
        return e;
    }
    if (*buf) {
        g_retired.push_back(*buf);
        g_retired_bytes += *bytes;
    }
    *buf = nb;
    *bytes = need;
    return hipSuccess;
}

hipError_t ensure_splitk_ws(size_t floats) {
    size_t wb = g_sk_ws_floats * sizeof(float);
    void* w = g_sk_ws;
    hipError_t e = grow(&w, &wb, floats * sizeof(float), false, "split-K workspace");
    g_sk_ws = static_cast<float*>(w);
    g_sk_ws_floats = wb / sizeof(float);
    return e;
}

// Launches projection p.  Split-K partials go to `fixed_ws` (capacity
// `fixed_floats`) when given -- the no-allocation entry point's scratch --
// else to the bridge's grow-only workspace.  -4 when p needs more than the
// fixed capacity.
int launch_ws(const qr::GemmParams& p0, float* fixed_ws, size_t fixed_floats) {
    qr::GemmParams p = p0;
    auto workspace = [&](size_t floats, float** ws) -> int {
        if (fixed_ws) {
            if (floats > fixed_floats) {
                char buf[160];
                snprintf(buf, sizeof(buf), "split-K partials need %zu floats, the fixed scratch holds %zu", floats,
                         fixed_floats);
                g_last_error = buf;
                return -4;
            }
            *ws = fixed_ws;
            return 0;
        }
        if (ensure_splitk_ws(floats) != hipSuccess) return staging_failed();
        *ws = g_sk_ws;
        return 0;
    };
    if (qr::skinny_supported(p)) {
        const size_t floats = qr::skinny_workspace_floats(p.M, p.N, p.K);
        float* ws = nullptr;
        if (int rc = workspace(floats ? floats : 1, &ws)) return rc;
        hipError_t e = qr::launch_gemm_skinny(p, ws, g_stream);
        if (e != hipSuccess) {
            set_error("launch_gemm_skinny", e);
            return -6;
        }
        return 0;
    }
    p.ksplit = qr::gemm_pick_ksplit(p);
    if (p.ksplit > 1) {
        if (int rc = workspace(qr::gemm_workspace_floats(p, p.ksplit), &p.ws)) return rc;
    }
    hipError_t e = qr::launch_gemm(p, g_stream);
    if (e != hipSuccess) {
        set_error("launch_gemm", e);
        return -6;
    }
    return 0;
}

int launch(const qr::GemmParams& p) { return launch_ws(p, nullptr, 0); }

int gemm_common(void* X, size_t Xb, void* W, size_t Wb, void* Y, size_t Yb, void* R, int format, uint32_t M,
                uint32_t K, uint32_t N, uint32_t head_D, bool ext) {
    if (!g_initialized) return -1;
    int rc = validate(X, Xb, W, Wb, Y, Yb, format, M, K, N, ext);
    if (rc) return rc;
    if (!has_kernels(format)) return -3;
    const size_t wbytes = qr::kernel_weight_bytes(format, K, N);
    std::lock_guard<std::mutex> lk(g_mu);
    void* dx = resolve(X, (size_t)M * K * 2, 16, true, false);
    void* dw = resolve(W, wbytes, 16, true, false);
    void* dr = R ? resolve(R, (size_t)M * N * 2, 2, true, false) : nullptr;
    void* dy = resolve(Y, (size_t)M * N * 2, 2, false, true);
    if (!dx || !dw || !dy || (R && !dr)) return staging_failed();
    qr::GemmParams p{};
    p.format = format;
    p.X = static_cast<const _Float16*>(dx);
    p.W = static_cast<const uint8_t*>(dw);
    p.W2 = nullptr;
    p.Y = static_cast<_Float16*>(dy);
    p.R = static_cast<const _Float16*>(dr);
    p.M = M; p.N = N; p.K = K;
    p.head_D = head_D;
    p.col_bytes = wbytes / N;
    return finish(launch(p));
}

// ---- scratch of the no-allocation projection entry point ----
// Split-K partials of m4_bridge_dispatch_gemm_noalloc live in this
// file-scope device array (32 MiB, held on every GPU the library runs on
// until the process ends): enough for every tiled launch (at most 256
// workgroups of at most 128 x 256 outputs, so ksplit * M * N <= 8 Mi).  In host code `scratch` names a host-side stand-in
// only: its device address, per device, comes from hipGetSymbolAddress at
// init and is the only handle host code passes on.  Nothing in it has to
// start at zero: every split writes all of its partials before the
// reduction kernel reads them.
constexpr size_t kScratchFloats = (size_t)8 << 20;
static __device__ __align__(256) float scratch[kScratchFloats];
constexpr int kMaxDevices = 64;
float* g_scratch[kMaxDevices] = {};

}  // namespace

extern "C" {

bool m4_bridge_init(const char* /*metallib_path*/) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_initialized) return true;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        g_last_error = "no HIP device";
        return false;
    }
    hipError_t e = hipGetDevice(&g_device);
    if (e == hipSuccess) e = hipSetDevice(g_device);
    if (e == hipSuccess) e = hipStreamCreate(&g_own_stream);
    if (e != hipSuccess) {
        set_error("init", e);
        return false;
    }
    g_stream = g_own_stream;
    if (g_device >= 0 && g_device < kMaxDevices && !g_scratch[g_device]) {
        void* sp = nullptr;
        const hipError_t se = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
        if (se == hipSuccess) {
            g_scratch[g_device] = static_cast<float*>(sp);
        } else {
            (void)hipGetLastError();  // the other entry points do not need it
            set_error("hipGetSymbolAddress(scratch)", se);
        }
    }
    g_initialized = true;
    return true;
}

size_t m4_bridge_get_expected_weight_bytes(int format, uint32_t K, uint32_t N) {
    return qr::expected_weight_bytes(format, K, N);
}

int m4_bridge_validate_gemm(const void* X, size_t Xb, const void* W, size_t Wb, const void* Y, size_t Yb,
                            int format, uint32_t M, uint32_t K, uint32_t N) {
    return validate(X, Xb, W, Wb, Y, Yb, format, M, K, N);
}

int m4_bridge_dispatch_gemm(void* X, size_t Xb, void* W, size_t Wb, void* Y, size_t Yb, int format, uint32_t M,
                            uint32_t K, uint32_t N) {
    return gemm_common(X, Xb, W, Wb, Y, Yb, nullptr, format, M, K, N, 0, false);
}

int m4_bridge_dispatch_gemm_noalloc(void* X, size_t Xb, void* W, size_t Wb, void* Y, size_t Yb, int format,
                                    uint32_t M, uint32_t K, uint32_t N) {
    if (!g_initialized) return -1;
    int rc = validate(X, Xb, W, Wb, Y, Yb, format, M, K, N);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    float* ws = (g_device >= 0 && g_device < kMaxDevices) ? g_scratch[g_device] : nullptr;
    if (!ws) {
        g_last_error = "no-allocation scratch unavailable on this device";
        return -6;
    }
    // no staging (it would allocate): device buffers only, X and W 16-byte aligned
    if (device_view(X) != X || device_view(W) != W || device_view(Y) != Y ||
        (reinterpret_cast<uintptr_t>(X) % 16) || (reinterpret_cast<uintptr_t>(W) % 16)) {
        g_last_error = "no-allocation projection: X, W and Y must be device memory, X and W 16-byte aligned";
        return -2;
    }
    const size_t wbytes = qr::kernel_weight_bytes(format, K, N);
    qr::GemmParams p{};
    p.format = format;
    p.X = static_cast<const _Float16*>(X);
    p.W = static_cast<const uint8_t*>(W);
    p.Y = static_cast<_Float16*>(Y);
    p.M = M; p.N = N; p.K = K;
    p.col_bytes = wbytes / N;
    return launch_ws(p, ws, kScratchFloats);
}

int m4_bridge_dispatch_router_gemm(void* X, size_t Xb, void* W, size_t Wb, void* Y, size_t Yb, int format,
                                   uint32_t M, uint32_t K, uint32_t N) {
    return gemm_common(X, Xb, W, Wb, Y, Yb, nullptr, format, M, K, N, 0, true);
}

int m4_bridge_dispatch_gemv(void* x, size_t xb, void* W, size_t Wb, void* y, size_t yb, int format, uint32_t K,
                            uint32_t N) {
    return m4_bridge_dispatch_gemm(x, xb, W, Wb, y, yb, format, 1, K, N);
}

int m4_bridge_dispatch_head_gemm(void* X, size_t Xb, void* W, size_t Wb, void* Y, size_t Yb, int format, uint32_t M,
                                 uint32_t H, uint32_t D, uint32_t K) {
    if (!g_initialized) return -1;
    if (H == 0 || D == 0) return -4;
    return gemm_common(X, Xb, W, Wb, Y, Yb, nullptr, format, M, K, H * D, D, true);
}

int m4_bridge_dispatch_router_kernel(const char* kernel_name, void* X, size_t Xb, void* W, size_t Wb, void* Y,
                                     size_t Yb, const uint32_t* dims, uint32_t ndims) {
    if (!g_initialized) return -1;
    if (!kernel_name || !dims) return -2;
    const std::string name(kernel_name);
    // The vector-ALU ternary kernels compute the same projection as the
    // matrix-core ones (quant_router_kernels.metal:934-1201); here both names
    // run the MFMA path.
    int format = -1;
    bool head = false;
    if (name == "quant_router_gemm_ternary_1_58_vec") {
        format = qr::QUANT_TERNARY_1_58;
    } else if (name == "quant_router_head_gemm_ternary_1_58_vec") {
        format = qr::QUANT_TERNARY_1_58;
        head = true;
    } else {
        auto& reg = qr::QuantRegistry::instance();
        for (qr::QuantFormat f : reg.available_formats()) {
            const qr::QuantCodecDescriptor* d = reg.get(f);
            if (!d) continue;
            if (d->gemm_kernel_name == name) format = (int)f;
            else if (d->head_gemm_kernel_name == name) { format = (int)f; head = true; }
            if (format >= 0) break;
        }
    }
    if (format < 0 || !has_kernels(format)) return -3;
    if (head) {  // constant slots M, H, D, K
        if (ndims != 4) return -4;
        return m4_bridge_dispatch_head_gemm(X, Xb, W, Wb, Y, Yb, format, dims[0], dims[1], dims[2], dims[3]);
    }
    if (ndims != 3) return -4;  // constant slots M, N, K
    return gemm_common(X, Xb, W, Wb, Y, Yb, nullptr, format, dims[0], dims[2], dims[1], 0, true);
}

int m4_bridge_dispatch_gemm_residual(void* X, size_t Xb, void* W, size_t Wb, void* R, size_t Rb, void* Y, size_t Yb,
                                     int format, uint32_t M, uint32_t K, uint32_t N) {
    if (!g_initialized) return -1;
    if (!R || (reinterpret_cast<uintptr_t>(R) % 2)) return -2;
    if (Rb < (size_t)M * N * 2) return -2;
    return gemm_common(X, Xb, W, Wb, Y, Yb, R, format, M, K, N, 0, true);
}

int m4_bridge_dispatch_swiglu(void* X, size_t Xb, void* Wg, size_t Wgb, void* Wu, size_t Wub, void* Out,
                              size_t Outb, int format, uint32_t M, uint32_t Nm, uint32_t K) {
    if (!g_initialized) return -1;
    int rc = validate(X, Xb, Wg, Wgb, Out, Outb, format, M, K, Nm, true);
    if (rc) return rc;
    if (!Wu) return -2;
    if (Wub < qr::kernel_weight_bytes(format, K, Nm)) return -2;
    const size_t wbytes = qr::kernel_weight_bytes(format, K, Nm);
    std::lock_guard<std::mutex> lk(g_mu);
    void* dx = resolve(X, (size_t)M * K * 2, 16, true, false);
    void* dg = resolve(Wg, wbytes, 16, true, false);
    void* du = resolve(Wu, wbytes, 16, true, false);
    void* dy = resolve(Out, (size_t)M * Nm * 2, 2, false, true);
    if (!dx || !dg || !du || !dy) return staging_failed();
    qr::GemmParams p{};
    p.format = format;
    p.X = static_cast<const _Float16*>(dx);
    p.W = static_cast<const uint8_t*>(dg);
    p.W2 = static_cast<const uint8_t*>(du);
    p.Y = static_cast<_Float16*>(dy);
    p.M = M; p.N = Nm; p.K = K;
    p.col_bytes = wbytes / Nm;
    return finish(launch(p));
}

int m4_bridge_quantize_kv_q8_0(void* src, size_t src_bytes, void* dst, size_t dst_bytes, uint64_t nblocks) {
    if (!g_initialized) return -1;
    if (!src || !dst) return -2;
    if ((reinterpret_cast<uintptr_t>(src) % 2) || (reinterpret_cast<uintptr_t>(dst) % 2)) return -2;
    if (nblocks == 0) return -4;
    if (src_bytes < nblocks * 64 || dst_bytes < nblocks * 34) return -2;
    std::lock_guard<std::mutex> lk(g_mu);
    void* ds = resolve(src, nblocks * 64, 16, true, false);
    void* dd = resolve(dst, nblocks * 34, 2, false, true);
    if (!ds || !dd) return staging_failed();
    hipError_t e = qr::launch_quantize_q8_0(static_cast<const _Float16*>(ds), static_cast<uint8_t*>(dd), nblocks,
                                            g_stream);
    if (e != hipSuccess) set_error("quantize_q8_0", e);
    return finish(e != hipSuccess ? -6 : 0);
}

int m4_bridge_dispatch_flash_attn_q8_0_gqa(void* Q, size_t Qb, void* Kq, size_t Kqb, void* Vq, size_t Vqb, void* O,
                                           size_t Ob, uint32_t H, uint32_t Hkv, uint32_t M, uint32_t D, float scale,
                                           int o_token_major) {
    if (!g_initialized) return -1;
    if (!Q || !Kq || !Vq || !O) return -2;
    if ((reinterpret_cast<uintptr_t>(Q) % 2) || (reinterpret_cast<uintptr_t>(O) % 2)) return -2;
    if (H == 0 || M == 0 || Hkv == 0 || H % Hkv || (D != 64 && D != 128)) return -4;
    const size_t n = (size_t)H * M * D, nk = (size_t)Hkv * M * D;
    if (Qb < n * 2 || Ob < n * 2 || Kqb < nk / 32 * 34 || Vqb < nk / 32 * 34) return -2;
    std::lock_guard<std::mutex> lk(g_mu);
    void* dq = resolve(Q, n * 2, 16, true, false);
    void* dk = resolve(Kq, nk / 32 * 34, 4, true, false);
    void* dv = resolve(Vq, nk / 32 * 34, 4, true, false);
    void* dout = resolve(O, n * 2, 8, false, true);
    if (!dq || !dk || !dv || !dout) return staging_failed();
    // Q8_0 -> dequantized fp16 K [Hkv, Mp, D] and V^T [Hkv, D, Mp] once, so the
    // attention kernel stages tiles without decoding them per query tile
    const uint32_t Mp = qr::kv_padded_len(M);
    const size_t half_bytes = (size_t)Hkv * Mp * D * 2;
    if (grow(&g_attn_ws, &g_attn_ws_bytes, 2 * half_bytes, false, "attention cache") != hipSuccess)
        return staging_failed();
    _Float16* kf = static_cast<_Float16*>(g_attn_ws);
    _Float16* vtf = kf + half_bytes / 2;
    hipError_t e = qr::launch_kv_prep(dk, dv, true, kf, vtf, Hkv, M, D, g_stream);
    qr::AttnParams p{static_cast<const _Float16*>(dq), static_cast<_Float16*>(dout), H, M, D, scale,
                     o_token_major ? 1 : 0, Hkv, kf, vtf, Mp};
    if (e == hipSuccess) e = qr::launch_flash_attn_q8_0(p, g_stream);
    if (e != hipSuccess) set_error("flash_attn_q8_0", e);
    return finish(e != hipSuccess ? -6 : 0);
}

int m4_bridge_dispatch_flash_attn_q8_0(void* Q, size_t Qb, void* Kq, size_t Kqb, void* Vq, size_t Vqb, void* O,
                                       size_t Ob, uint32_t H, uint32_t M, uint32_t D, float scale,
                                       int o_token_major) {
    return m4_bridge_dispatch_flash_attn_q8_0_gqa(Q, Qb, Kq, Kqb, Vq, Vqb, O, Ob, H, H, M, D, scale, o_token_major);
}

int m4_bridge_dequantize(void* W, size_t Wb, void* out, size_t outb, int format, uint32_t K, uint32_t N) {
    if (!g_initialized) return -1;
    if (!W || !out) return -2;
    if (!has_kernels(format)) return -3;
    if (K == 0 || N == 0 || K % 32) return -4;
    if ((format == 2 || format == 4 || format == 5) && K % 256) return -4;
    if (format == 7 && K % 128) return -4;
    if (format == qr::QUANT_MLX_4BIT_G64 && K % 64) return -4;
    const size_t wbytes = qr::kernel_weight_bytes(format, K, N);
    if (Wb < wbytes || outb < (size_t)N * K * 2) return -2;
    if (wbytes >= (1ull << 31)) return -4;
    std::lock_guard<std::mutex> lk(g_mu);
    void* dw = resolve(W, wbytes, 16, true, false);
    void* dout = resolve(out, (size_t)N * K * 2, 16, false, true);
    if (!dw || !dout) return staging_failed();
    hipError_t e = qr::launch_dequant(format, static_cast<const uint8_t*>(dw), static_cast<_Float16*>(dout), K, N,
                                      wbytes / N, g_stream);
    if (e != hipSuccess) set_error("dequant", e);
    return finish(e != hipSuccess ? -6 : 0);
}

int m4_bridge_prefill_layer(void* X, void* Wq, void* Wk, void* Wv, void* Wo, void* Wg, void* Wu, void* Wd,
                            void* Xout, int format, uint32_t M, uint32_t dm, uint32_t H, uint32_t D, uint32_t Nm,
                            float scale) {
    if (!g_initialized) return -1;
    if (!Wq || !Wk || !Wv || !Wo || !Wg || !Wu || !Wd) return -2;
    return m4_bridge_prefill_layer_ex(X, nullptr, Wq, Wk, Wv, Wo, nullptr, Wg, Wu, Wd, Xout, format, M, dm, H, H, D,
                                      Nm, scale, 1, 0.0f, 0, 10000.0f, 0, 0);
}

int m4_bridge_prefill_layer_ex(void* X, void* w_attn, void* Wq, void* Wk, void* Wv, void* Wo, void* w_ffn, void* Wg,
                               void* Wu, void* Wd, void* Xout, int format, uint32_t M, uint32_t dm, uint32_t Hq,
                               uint32_t Hkv, uint32_t D, uint32_t Nm, float scale, int norm_type, float eps,
                               int rope, float theta, uint32_t offset, int traditional) {
    return m4_bridge_prefill_layer_ex_kv(X, w_attn, Wq, Wk, Wv, Wo, w_ffn, Wg, Wu, Wd, Xout, nullptr, nullptr, format, M,
                                         dm, Hq, Hkv, D, Nm, scale, norm_type, eps, rope, theta, offset, traditional);
}

int m4_bridge_prefill_layer_ex_kv(void* X, void* w_attn, void* Wq, void* Wk, void* Wv, void* Wo, void* w_ffn, void* Wg,
                                  void* Wu, void* Wd, void* Xout, void* Kq_out, void* Vq_out, int format, uint32_t M,
                                  uint32_t dm, uint32_t Hq, uint32_t Hkv, uint32_t D, uint32_t Nm, float scale,
                                  int norm_type, float eps, int rope, float theta, uint32_t offset, int traditional) {
    if (!g_initialized) return -1;
    if ((Kq_out == nullptr) != (Vq_out == nullptr)) return -2;
    for (void* q : {Kq_out, Vq_out}) {
        if (!q) continue;
        void* d = device_view(q);
        if (!d || d != q || (reinterpret_cast<uintptr_t>(q) % 2)) return -2;  // device, 2-byte aligned blocks
    }
    void* ptrs[9] = {X, Wq, Wk, Wv, Wo, Wg, Wu, Wd, Xout};
    for (void* q : ptrs)
        if (!q) return -2;
    if (!has_kernels(format)) return -3;
    if ((w_attn || w_ffn) && norm_type != 1 && norm_type != 2) return -3;
    if (M == 0 || dm == 0 || Hq == 0 || Hkv == 0 || Hq % Hkv || Nm == 0 || (D != 64 && D != 128)) return -4;
    const uint32_t HQ = Hq * D, HK = Hkv * D;
    const uint32_t bs = qr::get_quant_info(static_cast<qr::QuantFormat>(format)).block_size;
    if (dm % bs || HQ % bs || Nm % bs || dm % 32 || HQ % 32 || Nm % 32) return -4;
    for (void* q : ptrs) {
        void* d = device_view(q);
        if (!d || d != q || (reinterpret_cast<uintptr_t>(q) % 16)) return -2;  // device, 16-byte aligned
    }
    for (void* q : {w_attn, w_ffn}) {
        if (!q) continue;
        void* d = device_view(q);
        if (!d || d != q || (reinterpret_cast<uintptr_t>(q) % 16)) return -2;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    const size_t nq = (size_t)M * HQ, nk = (size_t)M * HK;
    const uint32_t Mp = qr::kv_padded_len(M);
    const size_t kvf = (size_t)Hkv * Mp * D * 2;  // one dequantized fp16 working copy (K or V^T)
    const size_t kvq = nk / 32 * 34;              // the Q8_0 cache of K or V
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const bool norms = w_attn || w_ffn;
    const size_t need = 2 * al(nq * 2) + 2 * al(nk * 2) + 2 * al(kvf) + 2 * al(kvq) + al((size_t)M * dm * 2) +
                        al((size_t)M * Nm * 2) + (norms ? al((size_t)M * dm * 2) : 0);
    if (grow(&g_ws, &g_ws_bytes, need, false, "layer scratch") != hipSuccess) return -5;
    uint8_t* w = static_cast<uint8_t*>(g_ws);
    auto take = [&](size_t b) { uint8_t* r = w; w += al(b); return r; };
    _Float16* q = reinterpret_cast<_Float16*>(take(nq * 2));
    _Float16* k = reinterpret_cast<_Float16*>(take(nk * 2));
    _Float16* v = reinterpret_cast<_Float16*>(take(nk * 2));
    _Float16* kf = reinterpret_cast<_Float16*>(take(kvf));
    _Float16* vtf = reinterpret_cast<_Float16*>(take(kvf));
    uint8_t* kq = take(kvq);
    uint8_t* vq = take(kvq);
    if (Kq_out) {  // the caller keeps the Q8_0 KV cache
        kq = static_cast<uint8_t*>(Kq_out);
        vq = static_cast<uint8_t*>(Vq_out);
    }
    _Float16* o = reinterpret_cast<_Float16*>(take(nq * 2));
    _Float16* xm = reinterpret_cast<_Float16*>(take((size_t)M * dm * 2));
    _Float16* s = reinterpret_cast<_Float16*>(take((size_t)M * Nm * 2));
    _Float16* xn = norms ? reinterpret_cast<_Float16*>(take((size_t)M * dm * 2)) : nullptr;

    auto proj = [&](const void* A, const void* W, const void* W2, _Float16* Y, const _Float16* R, uint32_t N,
                    uint32_t Kd, uint32_t headD) {
        qr::GemmParams p{};
        p.format = format;
        p.X = static_cast<const _Float16*>(A);
        p.W = static_cast<const uint8_t*>(W);
        p.W2 = static_cast<const uint8_t*>(W2);
        p.Y = Y;
        p.R = R;
        p.M = M; p.N = N; p.K = Kd;
        p.head_D = headD;
        p.col_bytes = qr::kernel_weight_bytes(format, Kd, N) / N;
        return launch(p);
    };
    auto check = [&](hipError_t e, const char* what) {
        if (e == hipSuccess) return 0;
        set_error(what, e);
        return -6;
    };
    int rc = 0;
    const void* a = X;
    if (w_attn) {
        rc = check(qr::launch_rmsnorm(static_cast<const _Float16*>(X), static_cast<const _Float16*>(w_attn), xn, M, dm,
                                      eps, norm_type, g_stream), "layer rmsnorm");
        a = xn;
    }
    // Q, K, V: one grouped launch when the three fit one grid, else three
    if (!rc) {
        qr::GemmParams g{};
        g.format = format;
        g.X = static_cast<const _Float16*>(a);
        g.W = static_cast<const uint8_t*>(Wq);
        g.Y = q;
        g.M = M; g.N = HQ; g.K = dm;
        g.head_D = D;
        g.col_bytes = qr::kernel_weight_bytes(format, dm, HQ) / HQ;
        g.ngroups = 3;
        g.Wx[0] = static_cast<const uint8_t*>(Wk); g.Yx[0] = k; g.Nx[0] = HK;
        g.Wx[1] = static_cast<const uint8_t*>(Wv); g.Yx[1] = v; g.Nx[1] = HK;
        if (qr::gemm_grouped_ok(g)) {
            g.ksplit = 1;
            rc = check(qr::launch_gemm(g, g_stream), "layer qkv");
        } else {
            rc = proj(a, Wq, nullptr, q, nullptr, HQ, dm, D);
            rc = rc ? rc : proj(a, Wk, nullptr, k, nullptr, HK, dm, D);
            rc = rc ? rc : proj(a, Wv, nullptr, v, nullptr, HK, dm, D);
        }
    }
    if (!rc && rope) {
        rc = check(qr::launch_rope(q, Hq, M, D, theta, offset, traditional, g_stream), "layer rope");
        rc = rc ? rc : check(qr::launch_rope(k, Hkv, M, D, theta, offset, traditional, g_stream), "layer rope");
    }
    if (!rc) {
        // The Q8_0 KV cache (unified_prefill_engine.mm:548-572), written in
        // the same pass that dequantizes it into the attention kernel's fp16
        // K / V^T working copy (quantize + dequantize in registers).
        hipError_t e = qr::launch_kv_prep(k, v, false, kf, vtf, Hkv, M, D, g_stream, kq, vq);
        qr::AttnParams ap{q, o, Hq, M, D, scale, 1, Hkv, kf, vtf, Mp};
        if (e == hipSuccess) e = qr::launch_flash_attn_q8_0(ap, g_stream);
        rc = check(e, "layer attention");
    }
    rc = rc ? rc : proj(o, Wo, nullptr, xm, static_cast<const _Float16*>(X), dm, HQ, 0);
    a = xm;
    if (!rc && w_ffn) {
        rc = check(qr::launch_rmsnorm(xm, static_cast<const _Float16*>(w_ffn), xn, M, dm, eps, norm_type, g_stream),
                   "layer rmsnorm");
        a = xn;
    }
    rc = rc ? rc : proj(a, Wg, Wu, s, nullptr, Nm, dm, 0);
    rc = rc ? rc : proj(s, Wd, nullptr, static_cast<_Float16*>(Xout), xm, dm, Nm, 0);
    return rc;
}

int m4_bridge_rmsnorm(void* X, size_t Xb, void* W, size_t Wb, void* Y, size_t Yb, uint32_t M, uint32_t D, float eps,
                      int norm_type) {
    if (!g_initialized) return -1;
    if (!X || !W || !Y) return -2;
    if (norm_type != 1 && norm_type != 2) return -3;
    if (M == 0 || D == 0 || D % 8) return -4;
    if (Xb < (size_t)M * D * 2 || Yb < (size_t)M * D * 2 || Wb < (size_t)D * 2) return -2;
    std::lock_guard<std::mutex> lk(g_mu);
    void* dx = resolve(X, (size_t)M * D * 2, 16, true, false);
    void* dw = resolve(W, (size_t)D * 2, 16, true, false);
    void* dy = resolve(Y, (size_t)M * D * 2, 16, false, true);
    if (!dx || !dw || !dy) return staging_failed();
    hipError_t e = qr::launch_rmsnorm(static_cast<const _Float16*>(dx), static_cast<const _Float16*>(dw),
                                      static_cast<_Float16*>(dy), M, D, eps, norm_type, g_stream);
    if (e != hipSuccess) set_error("rmsnorm", e);
    return finish(e != hipSuccess ? -6 : 0);
}

int m4_bridge_rope(void* T, size_t Tb, uint32_t H, uint32_t M, uint32_t D, float theta, uint32_t offset,
                   int traditional) {
    if (!g_initialized) return -1;
    if (!T) return -2;
    if (H == 0 || M == 0 || D == 0 || D % 16 || !(theta > 0.0f)) return -4;
    const size_t n = (size_t)H * M * D * 2;
    if (Tb < n) return -2;
    std::lock_guard<std::mutex> lk(g_mu);
    void* dt = resolve(T, n, 16, true, true);
    if (!dt) return staging_failed();
    hipError_t e = qr::launch_rope(static_cast<_Float16*>(dt), H, M, D, theta, offset, traditional, g_stream);
    if (e != hipSuccess) set_error("rope", e);
    return finish(e != hipSuccess ? -6 : 0);
}

void m4_bridge_synchronize(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    sync_and_release();
}

double m4_bridge_get_uma_footprint_mb(void) {
    long pages = 0, rss = 0;
    FILE* f = fopen("/proc/self/statm", "r");
    if (f) {
        if (fscanf(f, "%ld %ld", &pages, &rss) != 2) rss = 0;
        fclose(f);
    }
    double host_mb = (double)rss * 4096.0 / (1024.0 * 1024.0);
    std::lock_guard<std::mutex> lk(g_mu);  // the byte counts change under concurrent dispatches
    return host_mb + (double)(g_ws_bytes + g_attn_ws_bytes + g_staged_bytes + g_pool_bytes + g_sk_ws_floats * 4 +
                              g_retired_bytes) /
                         (1024.0 * 1024.0);
}

bool m4_bridge_is_initialized(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return g_initialized;
}

void m4_bridge_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_initialized) return;
    sync_and_release();
    if (g_ws) (void)hipFree(g_ws);
    g_ws = nullptr;
    g_ws_bytes = 0;
    if (g_attn_ws) (void)hipFree(g_attn_ws);
    g_attn_ws = nullptr;
    g_attn_ws_bytes = 0;
    if (g_sk_ws) (void)hipFree(g_sk_ws);
    for (void* r : g_retired) (void)hipFree(r);
    g_retired.clear();
    for (auto& b : g_pool) (void)hipFree(b.first);
    g_pool.clear();
    g_pool_bytes = 0;
    g_retired_bytes = 0;
    g_sk_ws = nullptr;
    g_sk_ws_floats = 0;
    if (g_own_stream) (void)hipStreamDestroy(g_own_stream);
    g_own_stream = nullptr;
    g_stream = nullptr;
    g_initialized = false;
}

int m4_bridge_set_stream(void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_initialized) return -1;
    g_stream = stream ? static_cast<hipStream_t>(stream) : g_own_stream;
    return 0;
}

void* m4_bridge_get_stream(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return g_stream;
}

const char* m4_bridge_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"
