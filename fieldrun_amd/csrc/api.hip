// api.hip — the extern "C" boundary declared in include/frq.h.
//
// Owns device selection, streams, the per-context workspace and the one-time
// weight uploads, and dispatches Bundle::mm / expert_mm semantics
// (/root/reference/src/bundle.rs:644-919, 404-461) onto the gfx950 kernels:
//   int8, M == 1           -> fused quant + GEMV (one launch)
//   int8, 2 <= M <= 16     -> quant kernel + skinny MFMA kernel (weights
//                             streamed once; bit-exact epilogue)
//   int8, M >  16          -> quant kernel (blocked a8) + int8 MFMA GEMM
//   int4                   -> blocked W4A32 GEMV (M == 1) / batched kernel
// Every failure becomes an int status plus frq_last_error(); nothing throws.
#include <atomic>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "frq_internal.h"

using namespace frq;

struct frq_w {
    Weight w;
};
struct frq_moe_w {
    MoeBank b;
};
struct frq_ctx {
    int device = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    int* err = nullptr;  // device word: kernels atomically OR 1 on NaN input
};

// Scratch of frq_mm_dev_noalloc: one static array per GPU (each device that
// loads the library holds its own copy until the process ends).  Host code
// never uses the array's name as an address: frq_init resolves the device
// address once per device with hipGetSymbolAddress and keeps it in
// g_scratch_ptr, and only that pointer reaches kernels.
static __device__ __align__(256) char scratch[FRQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int FRQ_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[FRQ_MAX_DEVICES];  // scratch's address on each device, null until resolved

// With `dev` current: resolve scratch's device address once for this device.
hipError_t scratch_setup(int dev) {
    if (dev < 0 || dev >= FRQ_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev]) return hipSuccess;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
    return hipSuccess;
}

void* scratch_of(int dev) {
    if (dev < 0 || dev >= FRQ_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch_ptr[dev];
}

thread_local std::string g_err;
thread_local int g_code = FRQ_OK;

int fail(int code, const std::string& msg) {
    g_err = msg;
    g_code = code;
    return code;
}
int hip_fail(hipError_t e, const char* what) {
    return fail(FRQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define HIPCHK(expr, what)                          \
    do {                                            \
        hipError_t e_ = (expr);                     \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int d) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != d) (void)hipSetDevice(d);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

// Grow the context workspace to at least `bytes` (synchronises first).
int ws_reserve(frq_ctx* c, size_t bytes) {
    if (bytes <= c->ws_bytes) return FRQ_OK;
    HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->ws) (void)hipFree(c->ws);
    c->ws = nullptr;
    c->ws_bytes = 0;
    const size_t want = round_up(bytes + bytes / 4, 1 << 20);
    HIPCHK(hipMalloc(&c->ws, want), "hipMalloc(workspace)");
    c->ws_bytes = want;
    return FRQ_OK;
}

struct Carve {
    char* p;
    template <class T>
    T* take(size_t count) {
        T* r = reinterpret_cast<T*>(p);
        p += round_up(count * sizeof(T), 256);
        return r;
    }
};

// Decode batches (m <= 16) take the row-major a8 and the HBM-bound kernels;
// larger m the blocked a8 and the MFMA GEMM.
bool use_gemv(const Weight& w, size_t m) {
    (void)w;
    return m <= 16;
}

// Bytes of per-call scratch for an int8 linear of m rows (a second, row-major
// a8 when the GEMM's blocked a8 must also be returned to the host).
size_t i8_scratch_bytes(const Weight& w, size_t m, bool rowmajor_copy) {
    const size_t mp = round_up(m, FRQ_MALIGN);
    size_t b = round_up(mp * w.kp, 256) + round_up(mp * 4, 256) +
               2 * round_up(mp * FRQ_T * 4, 256);
    if (rowmajor_copy) b += round_up(m * w.kp, 256);
    if (!use_gemv(w, m)) b += round_up(gemm_ws_bytes(m, w.kp, w.np), 256);
    return b;
}

// The int8 linear on device pointers; scratch carved from `sc`.  With a8o
// set, *a8o is a row-major (pitch kp) copy of the quantised rows.
int run_i8(frq_ctx* c, const Weight& w, const float* d_a, size_t m, float* d_out,
           int32_t* d_acc, char* scratch, int8_t** a8o, float** sao,
           uint32_t** oio, float** ovo) {
    const bool gemm = !use_gemv(w, m);
    const size_t mp = round_up(m, FRQ_MALIGN);
    Carve cv{scratch};
    int8_t* a8 = cv.take<int8_t>(mp * w.kp);
    float* sa = cv.take<float>(mp);
    uint32_t* oi = cv.take<uint32_t>(mp * FRQ_T);
    float* ov = cv.take<float>(mp * FRQ_T);
    int8_t* a8rm = (gemm && a8o) ? cv.take<int8_t>(m * w.kp) : a8;
    void* gws = gemm ? cv.take<char>(gemm_ws_bytes(m, w.kp, w.np)) : nullptr;
    if (a8o) { *a8o = a8rm; *sao = sa; *oio = oi; *ovo = ov; }
    if (w.k == 0) {
        HIPCHK(hipMemsetAsync(d_out, 0, m * w.n * sizeof(float), c->stream), "hipMemsetAsync");
        if (d_acc) HIPCHK(hipMemsetAsync(d_acc, 0, m * w.n * sizeof(int32_t), c->stream), "hipMemsetAsync");
        return FRQ_OK;
    }
    if (m == 1 && linear_m1_ok(w, d_a)) {
        HIPCHK(launch_linear_m1(w, d_a, d_out, d_acc, a8o ? a8 : nullptr, sa, oi, ov, c->err, c->stream),
               "launch linear_m1");
    } else if (!gemm) {
        HIPCHK(launch_quant(d_a, m, w.k, w.kp, a8, sa, oi, ov, c->err, c->stream), "launch quant");
        if (m == 1)
            HIPCHK(launch_gemv_i8(w, m, a8, sa, oi, ov, d_out, d_acc, c->stream), "launch gemv_i8");
        else
            HIPCHK(launch_skinny_i8(w, m, a8, sa, oi, ov, d_out, d_acc, c->stream), "launch skinny_i8");
    } else {
        HIPCHK(launch_quant(d_a, m, w.k, w.kp, a8, sa, oi, ov, c->err, c->stream, mp), "launch quant");
        HIPCHK(launch_gemm_i8(w, m, a8, sa, oi, ov, d_out, d_acc, gws, c->stream), "launch gemm_i8");
        if (a8rm != a8)  // the same quantisation, row-major, for the caller
            HIPCHK(launch_quant(d_a, m, w.k, w.kp, a8rm, sa, oi, ov, c->err, c->stream), "launch quant");
    }
    return FRQ_OK;
}

bool rows_exact_ok(const frq_w* wh, size_t m) {
    const Weight& w = wh->w;
    return w.dtype == FRQ_DT_I8 && m > 16 && m <= 65535 && w.k > 0 && w.wblk && w.wkn && w.kp <= 20480 &&
           !use_gemv(w, m);
}

int rows_exact(frq_ctx* c, const frq_w* wh, const float* d_a, size_t m, float* d_out) {
    if (!rows_exact_ok(wh, m)) return fail(FRQ_ERR_ARG, "mm_i8_rows_exact: shape not supported");
    const Weight& w = wh->w;
    DeviceGuard g(c->device);
    const size_t base = i8_scratch_bytes(w, m, false);
    if (int rc = ws_reserve(c, base + round_up(m * w.n * sizeof(int32_t), 256))) return rc;
    const size_t mp = round_up(m, FRQ_MALIGN);
    Carve cv{(char*)c->ws};
    int8_t* a8 = cv.take<int8_t>(mp * w.kp);
    float* sa = cv.take<float>(mp);
    uint32_t* oi = cv.take<uint32_t>(mp * FRQ_T);
    float* ov = cv.take<float>(mp * FRQ_T);
    void* gws = cv.take<char>(gemm_ws_bytes(m, w.kp, w.np));
    int32_t* acc = reinterpret_cast<int32_t*>((char*)c->ws + base);
    HIPCHK(launch_quant(d_a, m, w.k, w.kp, a8, sa, oi, ov, c->err, c->stream, mp), "launch quant");
    HIPCHK(launch_gemm_i8(w, m, a8, sa, oi, ov, d_out, acc, gws, c->stream, true), "launch gemm_i8");
    HIPCHK(launch_i8_exact_epilogue(w, m, sa, oi, ov, acc, d_out, c->stream), "launch i8 epilogue");
    return FRQ_OK;
}

int check_err_word(frq_ctx* c) {
    int h = 0;
    HIPCHK(hipMemcpy(&h, c->err, sizeof(int), hipMemcpyDeviceToHost), "hipMemcpy(err)");
    if (h) {
        const int zero = 0;
        HIPCHK(hipMemcpy(c->err, &zero, sizeof(int), hipMemcpyHostToDevice), "hipMemcpy(err)");
        return fail(FRQ_ERR_NAN, "NaN in activations (the reference panics in partial_cmp().unwrap())");
    }
    return FRQ_OK;
}

int check_ctx(const frq_ctx* c) {
    if (!c) return fail(FRQ_ERR_ARG, "null context");
    return FRQ_OK;
}

__global__ void transpose_i8_kernel(const int8_t* __restrict__ src, int rows, int cols,
                                    size_t spitch, int8_t* __restrict__ dst, size_t dpitch) {
    __shared__ int8_t tile[64][65];
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
        const int r = i / 64, cc = i % 64;
        if (r0 + r < rows && c0 + cc < cols) tile[r][cc] = src[(size_t)(r0 + r) * spitch + c0 + cc];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
        const int cc = i / 64, r = i % 64;
        if (r0 + r < rows && c0 + cc < cols) dst[(size_t)(c0 + cc) * dpitch + r0 + r] = tile[r][cc];
    }
}

__global__ void f16_to_f32_kernel(const uint16_t* __restrict__ h, float* __restrict__ f, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        f[i] = h2f(h[i]);
}

hipError_t transpose(const int8_t* src, size_t rows, size_t cols, size_t spitch,
                     int8_t* dst, size_t dpitch, hipStream_t s) {
    if (!rows || !cols) return hipSuccess;
    dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
    transpose_i8_kernel<<<grid, dim3(256), 0, s>>>(src, (int)rows, (int)cols, spitch, dst, dpitch);
    return hipGetLastError();
}

void free_weight(Weight& w) {
    DeviceGuard g(w.device);
    if (w.wt) (void)hipFree(w.wt);
    if (w.wkn) (void)hipFree(w.wkn);
    if (w.wblk) (void)hipFree(w.wblk);
    if (w.scale) (void)hipFree(w.scale);
    if (w.q4) (void)hipFree(w.q4);
    if (w.s4) (void)hipFree(w.s4);
    if (w.q4raw) (void)hipFree(w.q4raw);
    if (w.s4raw) (void)hipFree(w.s4raw);
    if (w.rowp) (void)hipFree(w.rowp);
    if (w.q4a_sm) (void)hipFree(w.q4a_sm);
    w = Weight{};
}

// Allocate the padded int8 buffers of w (n, k set) and zero them.
int alloc_i8(frq_ctx* c, Weight& w) {
    w.kp = round_up(w.k, FRQ_KALIGN);
    w.np = round_up(w.n, FRQ_NALIGN);
    const size_t kpa = w.kp ? w.kp : FRQ_KALIGN;
    HIPCHK(hipMalloc(&w.wt, w.np * kpa), "hipMalloc(wt)");
    HIPCHK(hipMalloc(&w.wkn, w.np * kpa), "hipMalloc(wkn)");
    HIPCHK(hipMalloc(&w.wblk, w.np * kpa), "hipMalloc(wblk)");
    HIPCHK(hipMalloc(&w.scale, w.np * sizeof(float)), "hipMalloc(scale)");
    HIPCHK(hipMemsetAsync(w.wt, 0, w.np * kpa, c->stream), "hipMemsetAsync");
    HIPCHK(hipMemsetAsync(w.wkn, 0, w.np * kpa, c->stream), "hipMemsetAsync");
    HIPCHK(hipMemsetAsync(w.scale, 0, w.np * sizeof(float), c->stream), "hipMemsetAsync");
    return FRQ_OK;
}

}  // namespace

namespace frq {
int set_error(int code, const std::string& msg) { return fail(code, msg); }
int last_code() { return g_code; }
int ctx_device(const frq_ctx* c) { return c->device; }
int* ctx_err(frq_ctx* c) { return c->err; }
int ctx_ws(frq_ctx* c, size_t bytes, void** ws) {
    if (int rc = ws_reserve(c, bytes)) return rc;
    *ws = c->ws;
    return FRQ_OK;
}
int device_cus(int dev) {
    static std::atomic<int> cus[64];  // 0: not yet asked
    if (dev < 0 || dev >= 64) return 256;
    int v = cus[dev].load(std::memory_order_relaxed);
    if (v <= 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}
const Weight* weight_of(const frq_w* w) { return &w->w; }
bool i8_rows_exact_ok(const frq_w* w, size_t m) { return rows_exact_ok(w, m); }
int mm_i8_rows_exact(frq_ctx* c, const frq_w* w, const float* d_a, size_t m, float* d_out) {
    return rows_exact(c, w, d_a, m, d_out);
}
}  // namespace frq

extern "C" {

const char* frq_last_error(void) { return g_err.c_str(); }

const char* frq_version(void) { return "fieldrun_amd 0.1.0 (gfx950)"; }

int frq_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

frq_ctx* frq_init(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        fail(FRQ_ERR_NODEV, "no HIP device visible");
        return nullptr;
    }
    if (device < 0 || device >= n) {
        fail(FRQ_ERR_ARG, "device index out of range");
        return nullptr;
    }
    frq_ctx* c = new (std::nothrow) frq_ctx;
    if (!c) { fail(FRQ_ERR_ARG, "out of host memory"); return nullptr; }
    c->device = device;
    DeviceGuard g(device);
    hipError_t e = hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&c->err, 256);
    if (e == hipSuccess) e = hipMemset(c->err, 0, 256);
    if (e == hipSuccess) e = scratch_setup(device);
    if (e != hipSuccess) {
        hip_fail(e, "frq_init");
        if (c->err) (void)hipFree(c->err);
        if (c->own) (void)hipStreamDestroy(c->own);
        delete c;
        return nullptr;
    }
    c->stream = c->own;
    return c;
}

void frq_free(frq_ctx* c) {
    if (!c) return;
    DeviceGuard g(c->device);
    (void)hipStreamSynchronize(c->stream);
    if (c->ws) (void)hipFree(c->ws);
    if (c->err) (void)hipFree(c->err);
    if (c->own) (void)hipStreamDestroy(c->own);
    delete c;
}

int frq_set_stream(frq_ctx* c, void* s) {
    if (int rc = check_ctx(c)) return rc;
    c->stream = s ? (hipStream_t)s : c->own;
    return FRQ_OK;
}

void* frq_get_stream(frq_ctx* c) { return c ? (void*)c->stream : nullptr; }

int frq_sync(frq_ctx* c) {
    if (int rc = check_ctx(c)) return rc;
    DeviceGuard g(c->device);
    HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return check_err_word(c);
}

// ---- uploads ---------------------------------------------------------------

frq_w* frq_upload_i8(frq_ctx* c, const int8_t* wt_nk, const float* scale,
                     size_t n, size_t k) {
    if (check_ctx(c) || (!wt_nk && n * k) || (!scale && n)) {
        fail(FRQ_ERR_ARG, "frq_upload_i8: null argument");
        return nullptr;
    }
    DeviceGuard g(c->device);
    frq_w* h = new (std::nothrow) frq_w;
    if (!h) { fail(FRQ_ERR_ARG, "out of host memory"); return nullptr; }
    Weight& w = h->w;
    w.dtype = FRQ_DT_I8; w.device = c->device; w.n = n; w.k = k;
    int rc = alloc_i8(c, w);
    hipError_t e = hipSuccess;
    if (!rc && n && k)
        e = hipMemcpy2DAsync(w.wt, w.kp, wt_nk, k, k, n, hipMemcpyHostToDevice, c->stream);
    if (!rc && e == hipSuccess && n)
        e = hipMemcpyAsync(w.scale, scale, n * sizeof(float), hipMemcpyHostToDevice, c->stream);
    if (!rc && e == hipSuccess) e = transpose(w.wt, n, k, w.kp, w.wkn, w.np, c->stream);
    if (!rc && e == hipSuccess) e = launch_blockify(w.wt, w.np, w.np, w.kp, w.kp, w.wblk, c->stream);
    if (!rc && e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "frq_upload_i8");
    if (rc) { free_weight(w); delete h; return nullptr; }
    return h;
}

frq_w* frq_upload_i8_bundle(frq_ctx* c, const int8_t* w_kn,
                            const uint16_t* scale_f16, size_t k, size_t n) {
    if (check_ctx(c) || (!w_kn && n * k) || (!scale_f16 && n)) {
        fail(FRQ_ERR_ARG, "frq_upload_i8_bundle: null argument");
        return nullptr;
    }
    DeviceGuard g(c->device);
    frq_w* h = new (std::nothrow) frq_w;
    if (!h) { fail(FRQ_ERR_ARG, "out of host memory"); return nullptr; }
    Weight& w = h->w;
    w.dtype = FRQ_DT_I8; w.device = c->device; w.n = n; w.k = k;
    int rc = alloc_i8(c, w);
    uint16_t* hs = nullptr;
    hipError_t e = hipSuccess;
    // the (in, out) blob goes straight into wkn (pitch Np); wt is its transpose
    if (!rc && n && k)
        e = hipMemcpy2DAsync(w.wkn, w.np, w_kn, n, n, k, hipMemcpyHostToDevice, c->stream);
    if (!rc && e == hipSuccess) e = transpose(w.wkn, k, n, w.np, w.wt, w.kp, c->stream);
    if (!rc && e == hipSuccess) e = launch_blockify(w.wt, w.np, w.np, w.kp, w.kp, w.wblk, c->stream);
    if (!rc && e == hipSuccess && n) e = hipMalloc(&hs, n * sizeof(uint16_t));
    if (!rc && e == hipSuccess && n)
        e = hipMemcpyAsync(hs, scale_f16, n * sizeof(uint16_t), hipMemcpyHostToDevice, c->stream);
    if (!rc && e == hipSuccess && n) {
        f16_to_f32_kernel<<<dim3(64), dim3(256), 0, c->stream>>>(hs, w.scale, n);
        e = hipGetLastError();
    }
    if (!rc && e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (hs) (void)hipFree(hs);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "frq_upload_i8_bundle");
    if (rc) { free_weight(w); delete h; return nullptr; }
    return h;
}

frq_w* frq_upload_i4(frq_ctx* c, const uint8_t* packed,
                     const uint16_t* scale_f16, size_t n, size_t k, size_t g) {
    if (check_ctx(c) || g == 0 || (!packed && n * k) || (!scale_f16 && n * k)) {
        fail(FRQ_ERR_ARG, "frq_upload_i4: null argument or zero group");
        return nullptr;
    }
    DeviceGuard gd(c->device);
    frq_w* h = new (std::nothrow) frq_w;
    if (!h) { fail(FRQ_ERR_ARG, "out of host memory"); return nullptr; }
    Weight& w = h->w;
    w.dtype = FRQ_DT_I4; w.device = c->device; w.n = n; w.k = k; w.g = g;
    const size_t rb = (k + 1) / 2, ng = (k + g - 1) / g;
    hipError_t e = hipMalloc(&w.q4raw, n * rb + 16);
    if (e == hipSuccess) e = hipMalloc(&w.s4raw, n * ng * 2 + 16);
    if (e == hipSuccess && n * rb)
        e = hipMemcpyAsync(w.q4raw, packed, n * rb, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess && n * ng)
        e = hipMemcpyAsync(w.s4raw, scale_f16, n * ng * 2, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess && g == 32 && k % 32 == 0 && k > 0 && n > 0) {
        const size_t bytes = i4_blocked_bytes(n, k);  // scales: 1/8 of it
        e = hipMalloc(&w.q4, bytes);
        if (e == hipSuccess) e = hipMalloc(&w.s4, bytes / 8);
        if (e == hipSuccess) e = launch_i4_block(w.q4raw, w.s4raw, n, k, w.q4, w.s4, c->stream);
        if (e == hipSuccess) w.i4_blocked = 1;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        hip_fail(e, "frq_upload_i4");
        free_weight(w);
        delete h;
        return nullptr;
    }
    return h;
}

frq_w* frq_upload_q4a(frq_ctx* c, const uint8_t* packed, const uint16_t* scale_f16, const uint16_t* min_f16,
                      size_t n, size_t k, size_t g) {
    if (check_ctx(c) || g == 0 || (n * k && (!packed || !scale_f16 || !min_f16))) {
        fail(FRQ_ERR_ARG, "frq_upload_q4a: null argument or zero group");
        return nullptr;
    }
    DeviceGuard gd(c->device);
    frq_w* h = new (std::nothrow) frq_w;
    if (!h) { fail(FRQ_ERR_ARG, "out of host memory"); return nullptr; }
    Weight& w = h->w;
    w.dtype = FRQ_DT_Q4A; w.device = c->device; w.n = n; w.k = k; w.g = g;
    const size_t rb = (k + 1) / 2, ng = (k + g - 1) / g;
    w.rpitch = q4a_pitch(k);
    std::vector<uint32_t> sm(n * ng);
    for (size_t i = 0; i < n * ng; ++i) sm[i] = (uint32_t)scale_f16[i] | ((uint32_t)min_f16[i] << 16);
    hipError_t e = hipMalloc(&w.q4raw, n * w.rpitch + 16);
    if (e == hipSuccess) e = hipMalloc(&w.q4a_sm, n * ng * 4 + 16);
    if (e == hipSuccess) e = hipMemsetAsync(w.q4raw, 0, n * w.rpitch + 16, c->stream);
    if (e == hipSuccess && n * rb)
        e = hipMemcpy2DAsync(w.q4raw, w.rpitch, packed, rb, rb, n, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess && n * ng)
        e = hipMemcpyAsync(w.q4a_sm, sm.data(), n * ng * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);  // sm is released on return
    if (e != hipSuccess) {
        hip_fail(e, "frq_upload_q4a");
        free_weight(w);
        delete h;
        return nullptr;
    }
    return h;
}

frq_w* frq_upload_rows(frq_ctx* c, int dtype, const void* data, const float* scale, size_t rows,
                       size_t d) {
    if (check_ctx(c)) return nullptr;
    if (dtype != FRQ_DT_F32 && dtype != FRQ_DT_F16 && dtype != FRQ_DT_ROWI8) {
        fail(FRQ_ERR_DTYPE, "frq_upload_rows: dtype must be FRQ_DT_F32, FRQ_DT_F16 or FRQ_DT_ROWI8");
        return nullptr;
    }
    if ((!data && rows * d) || (dtype == FRQ_DT_ROWI8 && !scale && rows)) {
        fail(FRQ_ERR_ARG, "frq_upload_rows: null data or scale");
        return nullptr;
    }
    if (rows > (size_t)INT32_MAX || d > (size_t)INT32_MAX) {
        fail(FRQ_ERR_ARG, "frq_upload_rows: rows and d must fit in int32");
        return nullptr;
    }
    DeviceGuard gd(c->device);
    frq_w* h = new (std::nothrow) frq_w;
    if (!h) { fail(FRQ_ERR_ARG, "out of host memory"); return nullptr; }
    Weight& w = h->w;
    w.dtype = dtype; w.device = c->device; w.n = rows; w.k = d;
    const size_t es = dtype == FRQ_DT_F32 ? 4 : (dtype == FRQ_DT_F16 ? 2 : 1);
    w.rpitch = row_pitch(dtype, d);
    // at least one (zero) row: invalid subset ids read row 0 before scoring -inf
    const size_t bytes = (rows ? rows : 1) * w.rpitch + 128;
    hipError_t e = hipMalloc(&w.rowp, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(w.rowp, 0, bytes, c->stream);
    if (e == hipSuccess && rows * d)
        e = hipMemcpy2DAsync(w.rowp, w.rpitch, data, d * es, d * es, rows, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess && dtype == FRQ_DT_ROWI8) {
        e = hipMalloc(&w.scale, rows * 4 + 16);
        if (e == hipSuccess && rows)
            e = hipMemcpyAsync(w.scale, scale, rows * 4, hipMemcpyHostToDevice, c->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        hip_fail(e, "frq_upload_rows");
        free_weight(w);
        delete h;
        return nullptr;
    }
    return h;
}

void frq_w_free(frq_w* w) {
    if (!w) return;
    free_weight(w->w);
    delete w;
}

int frq_w_info(const frq_w* w, int* dtype, size_t* n, size_t* k, size_t* g) {
    if (!w) return fail(FRQ_ERR_ARG, "null weight");
    if (dtype) *dtype = w->w.dtype;
    if (n) *n = w->w.n;
    if (k) *k = w->w.k;
    if (g) *g = w->w.g;
    return FRQ_OK;
}

// ---- linears -----------------------------------------------------------------

int frq_mm_dev(frq_ctx* c, const frq_w* wh, const float* d_a, size_t m, float* d_out) {
    if (int rc = check_ctx(c)) return rc;
    if (!wh) return fail(FRQ_ERR_ARG, "null weight");
    const Weight& w = wh->w;
    if (w.device != c->device) return fail(FRQ_ERR_ARG, "weight lives on another device");
    if (m == 0 || w.n == 0) return FRQ_OK;
    if (!d_a || !d_out) return fail(FRQ_ERR_ARG, "null activation/output pointer");
    DeviceGuard g(c->device);
    if (w.dtype == FRQ_DT_I8) {
        if (int rc = ws_reserve(c, i8_scratch_bytes(w, m, false))) return rc;
        return run_i8(c, w, d_a, m, d_out, nullptr, (char*)c->ws, nullptr, nullptr, nullptr, nullptr);
    }
    if (w.dtype == FRQ_DT_I4) {
        if (int rc = ws_reserve(c, i4_ws_floats(w, m) * sizeof(float) + 256)) return rc;
        HIPCHK(launch_i4(w, m, d_a, d_out, (float*)c->ws, c->stream), "launch i4");
        return FRQ_OK;
    }
    if (w.dtype == FRQ_DT_Q4A) {
        HIPCHK(launch_q4a(w, m, d_a, d_out, c->stream), "launch q4a");
        return FRQ_OK;
    }
    return fail(FRQ_ERR_DTYPE, "unsupported weight dtype");
}

int frq_mm_dev_noalloc(frq_ctx* c, const frq_w* wh, const float* d_a, size_t m, float* d_out) {
    if (int rc = check_ctx(c)) return rc;
    if (!wh) return fail(FRQ_ERR_ARG, "null weight");
    const Weight& w = wh->w;
    if (w.device != c->device) return fail(FRQ_ERR_ARG, "weight lives on another device");
    if (m == 0 || w.n == 0) return FRQ_OK;
    if (!d_a || !d_out) return fail(FRQ_ERR_ARG, "null activation/output pointer");
    char* sp = static_cast<char*>(scratch_of(c->device));
    if (!sp) return fail(FRQ_ERR_HIP, "frq_mm_dev_noalloc: the static scratch of this device is not set up");
    auto too_big = [&](size_t need) {
        return fail(FRQ_ERR_ARG, "frq_mm_dev_noalloc: this call needs " + std::to_string(need) +
                                     " bytes of scratch, the static scratch holds " +
                                     std::to_string((size_t)FRQ_NOALLOC_SCRATCH_BYTES));
    };
    DeviceGuard g(c->device);
    if (w.dtype == FRQ_DT_I8) {
        const size_t need = i8_scratch_bytes(w, m, false);
        if (need > FRQ_NOALLOC_SCRATCH_BYTES) return too_big(need);
        return run_i8(c, w, d_a, m, d_out, nullptr, sp, nullptr, nullptr, nullptr, nullptr);
    }
    if (w.dtype == FRQ_DT_I4) {
        const size_t need = i4_ws_floats(w, m) * sizeof(float) + 256;
        if (need > FRQ_NOALLOC_SCRATCH_BYTES) return too_big(need);
        HIPCHK(launch_i4(w, m, d_a, d_out, reinterpret_cast<float*>(sp), c->stream), "launch i4");
        return FRQ_OK;
    }
    if (w.dtype == FRQ_DT_Q4A) {
        HIPCHK(launch_q4a(w, m, d_a, d_out, c->stream), "launch q4a");
        return FRQ_OK;
    }
    return fail(FRQ_ERR_DTYPE, "unsupported weight dtype");
}

size_t frq_quant_pitch(size_t k) { return round_up(k, FRQ_KALIGN); }

int frq_quant_i8_dev(frq_ctx* c, const float* d_a, size_t m, size_t k, int8_t* d_a8,
                     float* d_sa, uint32_t* d_oidx, float* d_oval) {
    if (int rc = check_ctx(c)) return rc;
    if (m == 0) return FRQ_OK;
    if ((!d_a && k) || !d_a8 || !d_sa || !d_oidx || !d_oval)
        return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    const size_t kp = round_up(k, FRQ_KALIGN);
    if (k == 0) {
        HIPCHK(hipMemsetAsync(d_oidx, 0, m * FRQ_T * 4, c->stream), "hipMemsetAsync");
        HIPCHK(hipMemsetAsync(d_oval, 0, m * FRQ_T * 4, c->stream), "hipMemsetAsync");
        return FRQ_OK;
    }
    HIPCHK(launch_quant(d_a, m, k, kp, d_a8, d_sa, d_oidx, d_oval, c->err, c->stream), "launch quant");
    return FRQ_OK;
}

int frq_mm_i8_q_dev(frq_ctx* c, const frq_w* wh, const int8_t* d_a8, const float* d_sa,
                    const uint32_t* d_oidx, const float* d_oval, size_t m, float* d_out) {
    if (int rc = check_ctx(c)) return rc;
    if (!wh) return fail(FRQ_ERR_ARG, "null weight");
    const Weight& w = wh->w;
    if (w.dtype != FRQ_DT_I8) return fail(FRQ_ERR_DTYPE, "frq_mm_i8_q_dev: not an int8 weight");
    if (w.device != c->device) return fail(FRQ_ERR_ARG, "weight lives on another device");
    if (m == 0 || w.n == 0) return FRQ_OK;
    if (!d_a8 || !d_sa || !d_oidx || !d_oval || !d_out) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    if (w.k == 0) {
        HIPCHK(hipMemsetAsync(d_out, 0, m * w.n * sizeof(float), c->stream), "hipMemsetAsync");
        return FRQ_OK;
    }
    if (use_gemv(w, m)) {
        if (m == 1)
            HIPCHK(launch_gemv_i8(w, m, d_a8, d_sa, d_oidx, d_oval, d_out, nullptr, c->stream), "launch gemv_i8");
        else
            HIPCHK(launch_skinny_i8(w, m, d_a8, d_sa, d_oidx, d_oval, d_out, nullptr, c->stream),
                   "launch skinny_i8");
        return FRQ_OK;
    }
    // the MFMA GEMM reads round_up(m, 128) rows of a8 in the blocked layout
    const size_t mp = round_up(m, FRQ_MALIGN);
    if (int rc = ws_reserve(c, round_up(mp * w.kp, 256) + gemm_ws_bytes(m, w.kp, w.np))) return rc;
    int8_t* a8 = (int8_t*)c->ws;
    void* gws = (char*)c->ws + round_up(mp * w.kp, 256);
    HIPCHK(launch_blockify(d_a8, m, mp, w.kp, w.kp, a8, c->stream), "launch blockify");
    HIPCHK(launch_gemm_i8(w, m, a8, d_sa, d_oidx, d_oval, d_out, nullptr, gws, c->stream), "launch gemm_i8");
    return FRQ_OK;
}

int frq_mm_i8_acc_dev(frq_ctx* c, const frq_w* wh, const int8_t* d_a8, size_t m, int32_t* d_acc) {
    if (int rc = check_ctx(c)) return rc;
    if (!wh) return fail(FRQ_ERR_ARG, "null weight");
    const Weight& w = wh->w;
    if (w.dtype != FRQ_DT_I8) return fail(FRQ_ERR_DTYPE, "frq_mm_i8_acc_dev: not an int8 weight");
    if (w.device != c->device) return fail(FRQ_ERR_ARG, "weight lives on another device");
    if (m == 0 || w.n == 0) return FRQ_OK;
    if (!d_a8 || !d_acc) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    if (w.k == 0) {
        HIPCHK(hipMemsetAsync(d_acc, 0, m * w.n * sizeof(int32_t), c->stream), "hipMemsetAsync");
        return FRQ_OK;
    }
    // the dot kernels need the quant's outputs only for their epilogues:
    // placeholders (sa = 1, no outliers) in the workspace, the sums to d_acc
    const bool gemm = rows_exact_ok(wh, m);
    const size_t mp = round_up(m, FRQ_MALIGN);
    const size_t base = round_up(mp * w.kp, 256) + round_up(mp * sizeof(float), 256) +
                        round_up(mp * FRQ_T * sizeof(uint32_t), 256) + round_up(mp * FRQ_T * sizeof(float), 256);
    const size_t gwb = gemm ? gemm_ws_bytes(m, w.kp, w.np) : 0;
    if (int rc = ws_reserve(c, base + gwb + round_up(m * w.n * sizeof(float), 256))) return rc;
    Carve cv{(char*)c->ws};
    int8_t* a8 = cv.take<int8_t>(mp * w.kp);
    float* sa = cv.take<float>(mp);
    uint32_t* oi = cv.take<uint32_t>(mp * FRQ_T);
    float* ov = cv.take<float>(mp * FRQ_T);
    void* gws = gemm ? cv.take<char>(gwb) : nullptr;
    float* out = cv.take<float>(m * w.n);
    HIPCHK(hipMemsetAsync(sa, 0, mp * sizeof(float), c->stream), "hipMemsetAsync");
    HIPCHK(hipMemsetAsync(oi, 0, mp * FRQ_T * sizeof(uint32_t), c->stream), "hipMemsetAsync");
    HIPCHK(hipMemsetAsync(ov, 0, mp * FRQ_T * sizeof(float), c->stream), "hipMemsetAsync");
    if (gemm) {
        HIPCHK(launch_blockify(d_a8, m, mp, w.kp, w.kp, a8, c->stream), "launch blockify");
        HIPCHK(launch_gemm_i8(w, m, a8, sa, oi, ov, out, d_acc, gws, c->stream, true), "launch gemm_i8");
    } else if (m == 1) {
        HIPCHK(launch_gemv_i8(w, m, d_a8, sa, oi, ov, out, d_acc, c->stream), "launch gemv_i8");
    } else if (m <= 16) {
        HIPCHK(launch_skinny_i8(w, m, d_a8, sa, oi, ov, out, d_acc, c->stream), "launch skinny_i8");
    } else {
        return fail(FRQ_ERR_ARG, "frq_mm_i8_acc_dev: shape not supported (K beyond 20480 at M > 16)");
    }
    return FRQ_OK;
}

static int mm_host(frq_ctx* c, const frq_w* wh, const float* a, size_t m, float* out,
                   int32_t* acc, int8_t* a8h, float* sah, uint32_t* oih, float* ovh) {
    if (int rc = check_ctx(c)) return rc;
    if (!wh) return fail(FRQ_ERR_ARG, "null weight");
    const Weight& w = wh->w;
    if (w.device != c->device) return fail(FRQ_ERR_ARG, "weight lives on another device");
    if (m == 0 || w.n == 0) return FRQ_OK;
    if ((!a && w.k) || !out) return fail(FRQ_ERR_ARG, "null activation/output pointer");
    DeviceGuard g(c->device);
    const bool i8 = w.dtype == FRQ_DT_I8;
    if (!i8 && w.dtype != FRQ_DT_I4 && w.dtype != FRQ_DT_Q4A) return fail(FRQ_ERR_DTYPE, "unsupported weight dtype");
    if (!i8 && (acc || a8h || sah || oih || ovh))
        return fail(FRQ_ERR_DTYPE, "debug outputs exist for int8 weights only");
    const size_t in_b = round_up(m * w.k * sizeof(float) + 16, 256);
    const size_t out_b = round_up(m * w.n * sizeof(float), 256);
    const size_t acc_b = acc ? round_up(m * w.n * sizeof(int32_t), 256) : 0;
    const size_t work = i8 ? i8_scratch_bytes(w, m, a8h && !use_gemv(w, m))
                           : round_up(i4_ws_floats(w, m) * sizeof(float) + 256, 256);
    if (int rc = ws_reserve(c, in_b + out_b + acc_b + work)) return rc;
    char* base = (char*)c->ws;
    float* d_a = (float*)base;
    float* d_out = (float*)(base + in_b);
    int32_t* d_acc = acc ? (int32_t*)(base + in_b + out_b) : nullptr;
    char* scratch = base + in_b + out_b + acc_b;
    if (m * w.k)
        HIPCHK(hipMemcpyAsync(d_a, a, m * w.k * sizeof(float), hipMemcpyHostToDevice, c->stream),
               "hipMemcpyAsync(a)");
    int8_t* a8 = nullptr; float* sa = nullptr; uint32_t* oi = nullptr; float* ov = nullptr;
    if (i8) {
        if (int rc = run_i8(c, w, d_a, m, d_out, d_acc, scratch, &a8, &sa, &oi, &ov)) return rc;
    } else if (w.dtype == FRQ_DT_Q4A) {
        HIPCHK(launch_q4a(w, m, d_a, d_out, c->stream), "launch q4a");
    } else {
        HIPCHK(launch_i4(w, m, d_a, d_out, (float*)scratch, c->stream), "launch i4");
    }
    HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (int rc = check_err_word(c)) return rc;
    HIPCHK(hipMemcpy(out, d_out, m * w.n * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy(out)");
    if (acc) HIPCHK(hipMemcpy(acc, d_acc, m * w.n * sizeof(int32_t), hipMemcpyDeviceToHost), "hipMemcpy(acc)");
    if (i8 && w.k) {
        if (a8h) HIPCHK(hipMemcpy2D(a8h, w.k, a8, w.kp, w.k, m, hipMemcpyDeviceToHost), "hipMemcpy2D(a8)");
        if (sah) HIPCHK(hipMemcpy(sah, sa, m * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy(sa)");
        if (oih) HIPCHK(hipMemcpy(oih, oi, m * FRQ_T * 4, hipMemcpyDeviceToHost), "hipMemcpy(oidx)");
        if (ovh) HIPCHK(hipMemcpy(ovh, ov, m * FRQ_T * 4, hipMemcpyDeviceToHost), "hipMemcpy(oval)");
    }
    return FRQ_OK;
}

int frq_mm(frq_ctx* c, const frq_w* w, const float* a, size_t m, float* out) {
    return mm_host(c, w, a, m, out, nullptr, nullptr, nullptr, nullptr, nullptr);
}

int frq_mm_i8_debug(frq_ctx* c, const frq_w* w, const float* a, size_t m, float* out,
                    int32_t* acc, int8_t* a8, float* sa, uint32_t* oidx, float* oval) {
    if (w && w->w.dtype != FRQ_DT_I8) return fail(FRQ_ERR_DTYPE, "frq_mm_i8_debug: not an int8 weight");
    return mm_host(c, w, a, m, out, acc, a8, sa, oidx, oval);
}

// ---- the unembed -------------------------------------------------------------

static int rowdot_check(frq_ctx* c, const frq_w* wh) {
    if (int rc = check_ctx(c)) return rc;
    if (!wh) return fail(FRQ_ERR_ARG, "null weight");
    const Weight& w = wh->w;
    if (w.dtype != FRQ_DT_F32 && w.dtype != FRQ_DT_F16 && w.dtype != FRQ_DT_ROWI8)
        return fail(FRQ_ERR_DTYPE, "rowdot_f32: not a row table (column-major quant unembed unsupported)");
    if (w.device != c->device) return fail(FRQ_ERR_ARG, "weight lives on another device");
    return FRQ_OK;
}

int frq_rowdot_f32_dev(frq_ctx* c, const frq_w* wh, const float* d_x, float* d_out) {
    if (int rc = rowdot_check(c, wh)) return rc;
    const Weight& w = wh->w;
    if (!w.n) return FRQ_OK;
    if ((!d_x && w.k) || !d_out) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    HIPCHK(launch_rowdot(w, d_x, nullptr, w.n, d_out, c->stream), "launch rowdot");
    return FRQ_OK;
}

int frq_rowdot_f32_subset_dev(frq_ctx* c, const frq_w* wh, const float* d_x, const int64_t* d_cand,
                              size_t ncand, float* d_out) {
    if (int rc = rowdot_check(c, wh)) return rc;
    const Weight& w = wh->w;
    if (!ncand) return FRQ_OK;
    if ((!d_x && w.k) || !d_cand || !d_out) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    HIPCHK(launch_rowdot(w, d_x, d_cand, ncand, d_out, c->stream), "launch rowdot");
    return FRQ_OK;
}

static int rowdot_host(frq_ctx* c, const frq_w* wh, const float* x, const int64_t* cand, size_t nout,
                       float* out) {
    if (int rc = rowdot_check(c, wh)) return rc;
    const Weight& w = wh->w;
    if (!nout) return FRQ_OK;
    if ((!x && w.k) || !out) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    const size_t xb = round_up(w.k * 4 + 16, 256), cb = cand ? round_up(nout * 8, 256) : 0;
    if (int rc = ws_reserve(c, xb + cb + round_up(nout * 4, 256))) return rc;
    char* base = (char*)c->ws;
    float* d_x = (float*)base;
    int64_t* d_cand = cand ? (int64_t*)(base + xb) : nullptr;
    float* d_out = (float*)(base + xb + cb);
    if (w.k) HIPCHK(hipMemcpyAsync(d_x, x, w.k * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(x)");
    if (cand) HIPCHK(hipMemcpyAsync(d_cand, cand, nout * 8, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(cand)");
    HIPCHK(launch_rowdot(w, d_x, d_cand, nout, d_out, c->stream), "launch rowdot");
    HIPCHK(hipMemcpyAsync(out, d_out, nout * 4, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(out)");
    HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return FRQ_OK;
}

int frq_rowdot_f32(frq_ctx* c, const frq_w* wh, const float* x, float* out) {
    if (int rc = rowdot_check(c, wh)) return rc;
    return rowdot_host(c, wh, x, nullptr, wh->w.n, out);
}

int frq_rowdot_f32_subset(frq_ctx* c, const frq_w* wh, const float* x, const int64_t* cand, size_t ncand,
                          float* out) {
    if (ncand && !cand) return fail(FRQ_ERR_ARG, "null candidate ids");
    return rowdot_host(c, wh, x, ncand ? cand : nullptr, ncand, out);
}

// ---- MoE -----------------------------------------------------------------------

frq_moe_w* frq_moe_upload_i8(frq_ctx* c, size_t n_exp, size_t d, size_t mi, int act,
                             const int8_t* const* gate, const float* const* gate_scale,
                             const int8_t* const* up, const float* const* up_scale,
                             const int8_t* const* down, const float* const* down_scale) {
    if (check_ctx(c) || !n_exp || !d || !mi || !gate || !gate_scale || !down || !down_scale ||
        (act == FRQ_ACT_SILU && (!up || !up_scale)) ||
        (act != FRQ_ACT_SILU && act != FRQ_ACT_GELU_TANH)) {
        fail(FRQ_ERR_ARG, "frq_moe_upload_i8: bad argument");
        return nullptr;
    }
    DeviceGuard g(c->device);
    frq_moe_w* h = new (std::nothrow) frq_moe_w;
    if (!h) { fail(FRQ_ERR_ARG, "out of host memory"); return nullptr; }
    MoeBank& b = h->b;
    b.device = c->device; b.n_exp = n_exp; b.d = d; b.mi = mi; b.act = act;
    b.gw = act == FRQ_ACT_SILU ? mi : 2 * mi;
    hipError_t e = hipMalloc(&b.gate, n_exp * d * b.gw);
    if (e == hipSuccess) e = hipMalloc(&b.gate_s, n_exp * b.gw * 4);
    if (e == hipSuccess) e = hipMalloc(&b.down, n_exp * mi * d);
    if (e == hipSuccess) e = hipMalloc(&b.down_s, n_exp * d * 4);
    if (e == hipSuccess && act == FRQ_ACT_SILU) e = hipMalloc(&b.up, n_exp * d * mi);
    if (e == hipSuccess && act == FRQ_ACT_SILU) e = hipMalloc(&b.up_s, n_exp * mi * 4);
    for (size_t x = 0; x < n_exp && e == hipSuccess; ++x) {
        if (!gate[x] || !gate_scale[x] || !down[x] || !down_scale[x] ||
            (act == FRQ_ACT_SILU && (!up[x] || !up_scale[x]))) {
            e = hipErrorInvalidValue;
            break;
        }
        e = hipMemcpyAsync(b.gate + x * d * b.gw, gate[x], d * b.gw, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(b.gate_s + x * b.gw, gate_scale[x], b.gw * 4, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(b.down + x * mi * d, down[x], mi * d, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(b.down_s + x * d, down_scale[x], d * 4, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess && act == FRQ_ACT_SILU) {
            e = hipMemcpyAsync(b.up + x * d * mi, up[x], d * mi, hipMemcpyHostToDevice, c->stream);
            if (e == hipSuccess) e = hipMemcpyAsync(b.up_s + x * mi, up_scale[x], mi * 4, hipMemcpyHostToDevice, c->stream);
        }
    }
    // blocked MFMA-operand copies for the digit GEMM
    b.kpd = round_up(d, 64);
    b.kpm = round_up(mi, 64);
    const size_t gwp = round_up(b.gw, 16), mip = round_up(mi, 16), dp = round_up(d, 16);
    if (e == hipSuccess) e = hipMalloc(&b.gate_b, n_exp * gwp * b.kpd);
    if (e == hipSuccess) e = launch_moe_block(b.gate, n_exp, d, b.gw, b.kpd, gwp, b.gate_b, c->stream);
    if (e == hipSuccess && act == FRQ_ACT_SILU) e = hipMalloc(&b.up_b, n_exp * mip * b.kpd);
    if (e == hipSuccess && act == FRQ_ACT_SILU)
        e = launch_moe_block(b.up, n_exp, d, mi, b.kpd, mip, b.up_b, c->stream);
    if (e == hipSuccess) e = hipMalloc(&b.down_b, n_exp * dp * b.kpm);
    if (e == hipSuccess) e = launch_moe_block(b.down, n_exp, mi, d, b.kpm, dp, b.down_b, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        hip_fail(e, "frq_moe_upload_i8");
        frq_moe_free(h);
        return nullptr;
    }
    return h;
}

// A bank whose experts are stored as i4, q4a, f16 or f32 (the arms of
// expert_f32, src/bundle.rs:404-454): each matrix of every expert copied as
// stored, plus the int4 MFMA operand copy where g % 32 == 0.
static frq_moe_w* moe_upload_ex(frq_ctx* c, int dtype, size_t n_exp, size_t d, size_t mi, int act, size_t g,
                                const void* const* gate, const uint16_t* const* gate_scale,
                                const uint16_t* const* gate_min, const void* const* up,
                                const uint16_t* const* up_scale, const uint16_t* const* up_min,
                                const void* const* down, const uint16_t* const* down_scale,
                                const uint16_t* const* down_min) {
    const bool q = dtype == FRQ_DT_I4 || dtype == FRQ_DT_Q4A;
    if (q && g == 0) {
        fail(FRQ_ERR_ARG, "frq_moe_upload: an i4 / q4a bank needs its group size");
        return nullptr;
    }
    DeviceGuard dg(c->device);
    frq_moe_w* h = new (std::nothrow) frq_moe_w;
    if (!h) { fail(FRQ_ERR_ARG, "out of host memory"); return nullptr; }
    MoeBank& b = h->b;
    b.device = c->device; b.n_exp = n_exp; b.d = d; b.mi = mi; b.act = act; b.dtype = dtype; b.g = q ? g : 0;
    b.gw = act == FRQ_ACT_SILU ? mi : 2 * mi;
    const bool mfma = dtype == FRQ_DT_I4 && g % 32 == 0;
    // digit rows of whole group quads for the int4 MFMA kernel (as the int8
    // bank's, 64-input blocks, otherwise)
    b.kpd = round_up(d, mfma ? 128 : 64);
    b.kpm = round_up(mi, mfma ? 128 : 64);
    hipError_t e = hipSuccess;
    auto one = [&](ExpMat& m, size_t in, size_t out, const void* const* raw, const uint16_t* const* sc,
                   const uint16_t* const* mn) {
        m.in = in;
        m.out = out;
        const size_t ng = q ? (in + g - 1) / g : 0;
        const size_t per = q ? out * ((in + 1) / 2) : in * out * (dtype == FRQ_DT_F16 ? 2 : 4);
        e = hipMalloc(&m.raw, n_exp * per);
        if (e == hipSuccess && q) e = hipMalloc(&m.sc, n_exp * out * ng * 2);
        if (e == hipSuccess && dtype == FRQ_DT_Q4A) e = hipMalloc(&m.mn, n_exp * out * ng * 2);
        for (size_t x = 0; x < n_exp && e == hipSuccess; ++x) {
            if (!raw[x] || (q && !sc[x]) || (dtype == FRQ_DT_Q4A && !mn[x])) {
                e = hipErrorInvalidValue;
                break;
            }
            e = hipMemcpyAsync((char*)m.raw + x * per, raw[x], per, hipMemcpyHostToDevice, c->stream);
            if (e == hipSuccess && q)
                e = hipMemcpyAsync(m.sc + x * out * ng, sc[x], out * ng * 2, hipMemcpyHostToDevice, c->stream);
            if (e == hipSuccess && dtype == FRQ_DT_Q4A)
                e = hipMemcpyAsync(m.mn + x * out * ng, mn[x], out * ng * 2, hipMemcpyHostToDevice, c->stream);
        }
        if (e == hipSuccess && mfma) {
            const size_t nrb = (out + 15) / 16, ng4 = (in + 127) / 128;
            e = hipMalloc(&m.q4e, n_exp * nrb * ng4 * 1024);
            if (e == hipSuccess) e = hipMalloc(&m.s4e, n_exp * nrb * ng4 * 128);
            if (e == hipSuccess) e = launch_moe_i4_block(m, n_exp, g, c->stream);
        }
    };
    one(b.mg, d, b.gw, gate, gate_scale, gate_min);
    if (e == hipSuccess && act == FRQ_ACT_SILU) one(b.mu, d, mi, up, up_scale, up_min);
    if (e == hipSuccess) one(b.md, mi, d, down, down_scale, down_min);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        hip_fail(e, "frq_moe_upload");
        frq_moe_free(h);
        return nullptr;
    }
    return h;
}

frq_moe_w* frq_moe_upload(frq_ctx* c, int dtype, size_t n_exp, size_t d, size_t mi, int act, size_t g,
                          const void* const* gate, const uint16_t* const* gate_scale,
                          const uint16_t* const* gate_min, const void* const* up, const uint16_t* const* up_scale,
                          const uint16_t* const* up_min, const void* const* down,
                          const uint16_t* const* down_scale, const uint16_t* const* down_min) {
    const bool silu_ = act == FRQ_ACT_SILU;
    if (check_ctx(c) || !n_exp || !d || !mi || !gate || !down || (silu_ && !up) ||
        (act != FRQ_ACT_SILU && act != FRQ_ACT_GELU_TANH)) {
        fail(FRQ_ERR_ARG, "frq_moe_upload: bad argument");
        return nullptr;
    }
    if (dtype == FRQ_DT_I8) {  // the int8 bank, its f16 scales upcast (arr1o)
        if (!gate_scale || !down_scale || (silu_ && !up_scale)) {
            fail(FRQ_ERR_ARG, "frq_moe_upload: an i8 bank needs its scales");
            return nullptr;
        }
        const size_t gw = silu_ ? mi : 2 * mi;
        std::vector<std::vector<float>> gs(n_exp), us(n_exp), ds(n_exp);
        std::vector<const float*> gsp(n_exp), usp(n_exp, nullptr), dsp(n_exp);
        std::vector<const int8_t*> gp(n_exp), upp(n_exp, nullptr), dpp(n_exp);
        auto up16 = [](const uint16_t* h16, size_t n, std::vector<float>& out) {
            out.resize(n);
            for (size_t i = 0; i < n; ++i) {  // the bundle's f16 arrays need not be 2-byte aligned
                uint16_t v;
                std::memcpy(&v, reinterpret_cast<const char*>(h16) + 2 * i, 2);
                out[i] = h2f_host(v);
            }
        };
        for (size_t x = 0; x < n_exp; ++x) {
            if (!gate_scale[x] || !down_scale[x] || (silu_ && !up_scale[x])) {
                fail(FRQ_ERR_ARG, "frq_moe_upload: null scale");
                return nullptr;
            }
            up16(gate_scale[x], gw, gs[x]);
            up16(down_scale[x], d, ds[x]);
            gsp[x] = gs[x].data();
            dsp[x] = ds[x].data();
            gp[x] = (const int8_t*)gate[x];
            dpp[x] = (const int8_t*)down[x];
            if (silu_) {
                up16(up_scale[x], mi, us[x]);
                usp[x] = us[x].data();
                upp[x] = (const int8_t*)up[x];
            }
        }
        return frq_moe_upload_i8(c, n_exp, d, mi, act, gp.data(), gsp.data(), silu_ ? upp.data() : nullptr,
                                 silu_ ? usp.data() : nullptr, dpp.data(), dsp.data());
    }
    if (dtype != FRQ_DT_I4 && dtype != FRQ_DT_Q4A && dtype != FRQ_DT_F16 && dtype != FRQ_DT_F32) {
        fail(FRQ_ERR_DTYPE, "frq_moe_upload: expert dtype must be i8, i4, q4a, f16 or f32");
        return nullptr;
    }
    return moe_upload_ex(c, dtype, n_exp, d, mi, act, g, gate, gate_scale, gate_min, up, up_scale, up_min, down,
                         down_scale, down_min);
}

void frq_moe_free(frq_moe_w* h) {
    if (!h) return;
    MoeBank& b = h->b;
    DeviceGuard g(b.device);
    for (void* p : {(void*)b.gate, (void*)b.gate_s, (void*)b.up, (void*)b.up_s, (void*)b.down, (void*)b.down_s,
                    (void*)b.gate_b, (void*)b.up_b, (void*)b.down_b})
        if (p) (void)hipFree(p);
    for (ExpMat* m : {&b.mg, &b.mu, &b.md})
        for (void* p : {m->raw, (void*)m->sc, (void*)m->mn, (void*)m->q4e, (void*)m->s4e})
            if (p) (void)hipFree(p);
    delete h;
}

int frq_moe_info(const frq_moe_w* h, int* dtype, size_t* n_exp, size_t* d, size_t* mi, size_t* g) {
    if (!h) return fail(FRQ_ERR_ARG, "null MoE bank");
    if (dtype) *dtype = h->b.dtype;
    if (n_exp) *n_exp = h->b.n_exp;
    if (d) *d = h->b.d;
    if (mi) *mi = h->b.mi;
    if (g) *g = h->b.g;
    return FRQ_OK;
}

int frq_moe_dev(frq_ctx* c, const frq_moe_w* h, const float* d_x, size_t T,
                const float* d_logits, size_t topk, int norm_topk, const float* d_pes,
                float* d_out) {
    if (int rc = check_ctx(c)) return rc;
    if (!h) return fail(FRQ_ERR_ARG, "null MoE bank");
    const MoeBank& b = h->b;
    if (b.device != c->device) return fail(FRQ_ERR_ARG, "MoE bank lives on another device");
    if (topk == 0 || topk > b.n_exp) return fail(FRQ_ERR_ARG, "topk must be in [1, n_exp]");
    if (topk > 256) return fail(FRQ_ERR_ARG, "topk above 256 slots a token");
    if (T == 0) return FRQ_OK;
    if (!d_x || !d_logits || !d_out) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    if (int rc = ws_reserve(c, moe_ws_bytes(b, T, topk))) return rc;
    HIPCHK(launch_moe(b, d_x, T, d_logits, topk, norm_topk, d_pes, d_out, c->ws, c->err, c->stream),
           "launch moe");
    return FRQ_OK;
}

int frq_moe(frq_ctx* c, const frq_moe_w* h, const float* x, size_t T, const float* logits,
            size_t topk, int norm_topk, const float* pes, float* out) {
    if (int rc = check_ctx(c)) return rc;
    if (!h) return fail(FRQ_ERR_ARG, "null MoE bank");
    const MoeBank& b = h->b;
    if (topk == 0 || topk > b.n_exp) return fail(FRQ_ERR_ARG, "topk must be in [1, n_exp]");
    if (topk > 256) return fail(FRQ_ERR_ARG, "topk above 256 slots a token");
    if (T == 0) return FRQ_OK;
    if (!x || !logits || !out) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    const size_t xb = round_up(T * b.d * 4, 256), lb = round_up(T * b.n_exp * 4, 256);
    const size_t pb = pes ? round_up(b.n_exp * 4, 256) : 0;
    const size_t wsb = moe_ws_bytes(b, T, topk);
    if (int rc = ws_reserve(c, xb * 2 + lb + pb + wsb)) return rc;
    char* base = (char*)c->ws;
    float* dx = (float*)base;
    float* dout = (float*)(base + xb);
    float* dl = (float*)(base + 2 * xb);
    float* dp = pes ? (float*)(base + 2 * xb + lb) : nullptr;
    void* wsp = base + 2 * xb + lb + pb;
    HIPCHK(hipMemcpyAsync(dx, x, T * b.d * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    HIPCHK(hipMemcpyAsync(dl, logits, T * b.n_exp * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    if (pes) HIPCHK(hipMemcpyAsync(dp, pes, b.n_exp * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    HIPCHK(launch_moe(b, dx, T, dl, topk, norm_topk, dp, dout, wsp, c->err, c->stream), "launch moe");
    HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (int rc = check_err_word(c)) return rc;
    HIPCHK(hipMemcpy(out, dout, T * b.d * 4, hipMemcpyDeviceToHost), "hipMemcpy(out)");
    return FRQ_OK;
}

int frq_moe_route(frq_ctx* c, const float* logits, size_t T, size_t E, size_t topk,
                  int norm_topk, const float* pes, int32_t* sel, float* w) {
    if (int rc = check_ctx(c)) return rc;
    if (topk == 0 || topk > E) return fail(FRQ_ERR_ARG, "topk must be in [1, E]");
    if (T == 0) return FRQ_OK;
    if (!logits || !sel || !w) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    const size_t lb = round_up(T * E * 4, 256), pb = round_up(E * 4, 256);
    const size_t sb = round_up(T * topk * 4, 256);
    if (int rc = ws_reserve(c, lb + pb + 2 * sb)) return rc;
    char* base = (char*)c->ws;
    float* dl = (float*)base;
    float* dp = pes ? (float*)(base + lb) : nullptr;
    int32_t* ds = (int32_t*)(base + lb + pb);
    float* dw = (float*)(base + lb + pb + sb);
    HIPCHK(hipMemcpyAsync(dl, logits, T * E * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    if (pes) HIPCHK(hipMemcpyAsync(dp, pes, E * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    HIPCHK(launch_moe_route(dl, T, E, topk, norm_topk, dp, ds, dw, c->err, c->stream), "launch route");
    HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (int rc = check_err_word(c)) return rc;
    HIPCHK(hipMemcpy(sel, ds, T * topk * 4, hipMemcpyDeviceToHost), "hipMemcpy(sel)");
    HIPCHK(hipMemcpy(w, dw, T * topk * 4, hipMemcpyDeviceToHost), "hipMemcpy(w)");
    return FRQ_OK;
}

int frq_expert_mm(frq_ctx* c, const frq_moe_w* h, int which, size_t e, const float* x,
                  size_t m, float* y) {
    if (int rc = check_ctx(c)) return rc;
    if (!h) return fail(FRQ_ERR_ARG, "null MoE bank");
    const MoeBank& b = h->b;
    if (e >= b.n_exp) return fail(FRQ_ERR_MISSING, "expert index out of range");
    const int8_t* q = nullptr;
    const float* s = nullptr;
    const ExpMat* mt = nullptr;
    size_t inp, out;
    const bool ex = b.dtype != FRQ_DT_I8;
    if (which == 0) {
        q = b.gate + e * b.d * b.gw; s = b.gate_s + e * b.gw; inp = b.d; out = b.gw; mt = &b.mg;
    } else if (which == 1 && b.act == FRQ_ACT_SILU) {
        q = b.up + e * b.d * b.mi; s = b.up_s + e * b.mi; inp = b.d; out = b.mi; mt = &b.mu;
    } else if (which == 2) {
        q = b.down + e * b.mi * b.d; s = b.down_s + e * b.d; inp = b.mi; out = b.d; mt = &b.md;
    } else {
        return fail(FRQ_ERR_MISSING, "no such expert bank");
    }
    if (m == 0) return FRQ_OK;
    if (!x || !y) return fail(FRQ_ERR_ARG, "null pointer");
    DeviceGuard g(c->device);
    const size_t xb = round_up(m * inp * 4, 256);
    if (int rc = ws_reserve(c, xb + m * out * 4)) return rc;
    float* dx = (float*)c->ws;
    float* dy = (float*)((char*)c->ws + xb);
    HIPCHK(hipMemcpyAsync(dx, x, m * inp * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    if (ex) HIPCHK(launch_expert_mm_ex(b, *mt, e, dx, m, dy, c->stream), "launch expert_mm");
    else HIPCHK(launch_expert_mm(q, s, inp, out, dx, m, dy, c->stream), "launch expert_mm");
    HIPCHK(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    HIPCHK(hipMemcpy(y, dy, m * out * 4, hipMemcpyDeviceToHost), "hipMemcpy(y)");
    return FRQ_OK;
}

}  // extern "C"
