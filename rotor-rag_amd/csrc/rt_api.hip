// C ABI of librotor_hip.so (declared in include/rotor_hip.h).
//
// The reference's GPU plug-in object (src/rotor/gpu_ternary.py:73-208) becomes an
// opaque context plus device-resident weight handles; every entry point returns a
// status code and leaves a thread-local message instead of raising
// (src/rotor/gpu_layers.py:18-25 latches on exceptions).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/rotor_hip.h"
#include "rt_internal.h"
#include "rt_rowquant.h"

using namespace rt;

namespace {

thread_local std::string g_err = "";

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(RT_EHIP, std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

#define RT_HIP(call)                                   \
    do {                                               \
        hipError_t _e = (call);                        \
        if (_e != hipSuccess) return hip_fail(_e, #call); \
    } while (0)

// Keeps the device current for the scope of an entry point.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Device buffer that only grows.  Work enqueued earlier (on whichever stream the context
// had then) may still read the old buffer, so the device is synchronised before it is
// freed; growth happens only when a call needs more rows than any call before it.
struct Scratch {
    void* p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t need) {
        if (need <= bytes) return hipSuccess;
        if (p) {
            hipError_t e = hipDeviceSynchronize();
            if (e != hipSuccess) return e;
            e = hipFree(p);
            if (e != hipSuccess) return e;
            p = nullptr;
            bytes = 0;
        }
        size_t cap = need < 4096 ? 4096 : need;
        hipError_t e = hipMalloc(&p, cap);
        if (e == hipSuccess) bytes = cap;
        return e;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
};

}  // namespace

// ---- static scratch of the allocation-free entry point ----------------------------------
// rt_linear_f32_noalloc stages its quantised activations here instead of in a context's
// growing buffer, for callers that cannot allocate.  Every device holds its own copy from
// the module load until the process ends.  In host code `scratch` is only a stand-in
// symbol, not a device address: the address is resolved per device with
// hipGetSymbolAddress (device current) and only that pointer is used.
static_assert(RT_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
static __device__ __align__(256) unsigned char scratch[RT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device `dev`, resolved once per device.
hipError_t noalloc_scratch(int dev, void** out) {
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        addr[dev] = p;
    }
    *out = addr[dev];
    return hipSuccess;
}

// Once per device `dev` (current): the kernels' function attributes, so that no launch
// (e.g. the first one of a shape inside a stream capture) makes a function-attribute call.
hipError_t prepare_device(int dev) {
    static std::mutex mu;
    static bool done[kMaxDevices] = {};
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (done[dev]) return hipSuccess;
    hipError_t e = gemm_prepare_device();
    if (e == hipSuccess) e = model_prepare_device();
    if (e == hipSuccess) done[dev] = true;
    return e;
}

}  // namespace

struct rt_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    Scratch act;  // qx [Mpad][Kp] followed by sx [Mpad]
    int8_t* noalloc = nullptr;  // this device's `scratch` (rt_linear_f32_noalloc)
};

struct rt_weights {
    int device = 0;
    int N = 0, K = 0, Kp = 0, C = 0, Np = 0;
    float scale = 1.0f;
    v4u* tiles = nullptr;
    size_t bytes = 0;
};

struct rt_plan {
    int device = 0;
    int G = 0, M = 0, Mpad = 0, mt = 1, total_rb = 0, U = 0;
    GemvShape shape{};
    GemvProb* dev_probs = nullptr;   // [G]
    int* dev_rb2p = nullptr;         // [total_rb]
    QuantProb* dev_quant = nullptr;  // [U]
    void* act = nullptr;             // quantised activations of the U distinct inputs
    std::vector<GemvProb> probs;
    std::vector<QuantProb> quant;
    std::vector<GemmArgs> gemms;     // M > kGemvMaxM: one MFMA GEMM launch per problem
    GemmArgs* dev_gemms = nullptr;   // M > 8: the problems of one grouped launch [G]
    int* dev_tile2p = nullptr;       // M > 64: problem of every tile of that launch
    int gemm_cfg = 0, gemm_tiles = 0;  // M > 64: tile shape, tiles over all problems
    bool pair_gemm = false;            // rt_plan_create_act_gate_up: tiles whose waves pair columns
    int gemm_units = 0;              // 8 < M <= 64: workgroups of the split-K launch (parts x row blocks)
    int* dev_unit2d = nullptr;       // 8 < M <= 64: descriptor of every unit
    std::vector<int> gemm_bnd;       // M > 8: first unit (tile) of descriptors 1.. (launch arguments)
    int* gemm_cnt = nullptr;         // split problems: arrivals per row block (zero between launches)
    int* gemm_ws = nullptr;          // split problems: int32 partial tiles
    std::vector<const rt_act*> acts; // plans over caller-quantised activations
    bool fused = false;              // M = 1, input quantised in the GEMV prologue
    QuantProb pro{};
    // rt_plan_run of an M = 1 plan over fp32 inputs: 1 the one shared input is quantised in
    // the KSPLIT prologue (pro), 2 every problem's own input in the ROWS prologue
    // (run_shape); 0 a quantiser launch, then the GEMV
    int run_pro = 0;
    GemvShape run_shape{};
    float* pair_a = nullptr;      // gate/up pair plan: relu(g)^2 * u [N / 2]
    double* pair_ssq = nullptr;   // its sum of squares per 32 outputs
    double* out_ssq = nullptr;    // rt_plan_set_output_ssq: f64 sums of squares per 32 outputs
    float* pair_g = nullptr;      // optional g, u [N / 2]
    float* pair_u = nullptr;
    float pair_sg = 1.0f, pair_su = 1.0f;  // gate and up scales
    int quant_maxK = 0;  // > 0: every quant problem takes the vectorised row kernel (largest K)
    // rt_plan_attach_attention: the decode attention partials run in rt_plan_run's launch
    bool att_on = false;
    AttnTail att{};
    int att_Hkv = 0, att_hd = 0;
    void* att_mem = nullptr;  // tagged outputs, epoch, done, err
    size_t att_bytes = 0;
};

struct rt_act {
    int device = 0;
    int Mcap = 0, K = 0, Kp = 0, Mpad_cap = 0;
    int M = 0;      // tokens held (set by the last quantise call)
    int Mpad = 0;   // rows valid for the GEMV/GEMM of M tokens (zero-filled past M)
    int8_t* qx = nullptr;
    float* sx = nullptr;
    void* mem = nullptr;
};

// Rows the matrix kernels read for M tokens: GEMV tokens per workgroup, or GEMM tile rows.
static int act_rows(int M) { return M > kGemvMaxM ? round_up(M, gemm_bm(M)) : round_up(M, gemv_mt(M)); }

extern "C" {

const char* rt_last_error(void) { return g_err.c_str(); }

int rt_version(void) { return 108; }

int rt_device_count(int* n) {
    if (!n) return fail(RT_EINVAL, "rt_device_count: n is NULL");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    *n = e == hipSuccess ? c : 0;
    return RT_OK;
}

int rt_ctx_create(int device, rt_ctx** out) {
    if (!out) return fail(RT_EINVAL, "rt_ctx_create: out is NULL");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(RT_ENODEV, "rt_ctx_create: no HIP device visible");
    if (device < 0 || device >= n) return fail(RT_EINVAL, "rt_ctx_create: device index out of range");
    hipDeviceProp_t prop;
    RT_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(RT_ENODEV, std::string("rt_ctx_create: device is ") + prop.gcnArchName +
                                   ", this library is built for gfx950 only");
    RT_HIP(hipSetDevice(device));
    void* sp = nullptr;
    RT_HIP(noalloc_scratch(device, &sp));
    RT_HIP(prepare_device(device));
    rt_ctx* c = new rt_ctx();
    c->device = device;
    c->noalloc = static_cast<int8_t*>(sp);
    *out = c;
    return RT_OK;
}

int rt_ctx_destroy(rt_ctx* ctx) {
    if (!ctx) return RT_OK;
    DeviceGuard g(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream); else (void)hipDeviceSynchronize();
    ctx->act.release();
    delete ctx;
    return RT_OK;
}

int rt_ctx_set_stream(rt_ctx* ctx, void* hip_stream) {
    if (!ctx) return fail(RT_EINVAL, "rt_ctx_set_stream: ctx is NULL");
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    return RT_OK;
}

int rt_sync(rt_ctx* ctx) {
    if (!ctx) return fail(RT_EINVAL, "rt_sync: ctx is NULL");
    DeviceGuard g(ctx->device);
    RT_HIP(hipStreamSynchronize(ctx->stream));
    return RT_OK;
}

static int weights_alloc(rt_ctx* ctx, int N, int K, float scale, rt_weights** out) {
    if (!ctx || !out) return fail(RT_EINVAL, "rt_weights_upload: ctx/out is NULL");
    if (N <= 0 || K <= 0) return fail(RT_EINVAL, "rt_weights_upload: N and K must be positive");
    // K <= 2^22 keeps the GEMV's int32 partial sums (4 g x over half the row, device code
    // g in 0..2, |x| <= 128) in range
    if ((long long)K > (1LL << 22) || (long long)N > (1LL << 26))
        return fail(RT_EINVAL, "rt_weights_upload: N or K too large (N <= 2^26, K <= 2^22)");
    rt_weights* w = new rt_weights();
    w->device = ctx->device;
    w->N = N;
    w->K = K;
    w->Kp = round_up(K, kChunk);
    w->C = w->Kp / kChunk;
    w->Np = round_up(N, kRowBlock);
    w->scale = scale;
    w->bytes = (size_t)w->Np * w->Kp / 4;
    hipError_t e = hipMalloc(&w->tiles, w->bytes + kTileSlack);
    if (e == hipSuccess) e = hipMemsetAsync(reinterpret_cast<char*>(w->tiles) + w->bytes, 0, kTileSlack, ctx->stream);
    if (e != hipSuccess) {
        if (w->tiles) (void)hipFree(w->tiles);
        delete w;
        return fail(RT_ENOMEM, std::string("rt_weights_upload: hipMalloc failed: ") + hipGetErrorName(e));
    }
    *out = w;
    return RT_OK;
}

int rt_weights_upload_device(rt_ctx* ctx, const uint8_t* rotor_dev, int N, int K, float scale, rt_weights** out) {
    if (!rotor_dev) return fail(RT_EINVAL, "rt_weights_upload_device: source is NULL");
    DeviceGuard g(ctx ? ctx->device : 0);
    int rc = weights_alloc(ctx, N, K, scale, out);
    if (rc) return rc;
    hipError_t e = launch_relayout(rotor_dev, N, K, (*out)->tiles, ctx->stream);
    if (e != hipSuccess) {
        rt_weights_free(*out);
        *out = nullptr;
        return hip_fail(e, "relayout launch");
    }
    return RT_OK;
}

int rt_weights_upload(rt_ctx* ctx, const uint8_t* rotor_host, int N, int K, float scale, rt_weights** out) {
    if (!rotor_host) return fail(RT_EINVAL, "rt_weights_upload: source is NULL");
    if (!ctx) return fail(RT_EINVAL, "rt_weights_upload: ctx is NULL");
    DeviceGuard g(ctx->device);
    int rc = weights_alloc(ctx, N, K, scale, out);
    if (rc) return rc;
    const size_t src_bytes = (size_t)N * ((K + 3) / 4);
    uint8_t* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, src_bytes);
    if (e == hipSuccess) e = hipMemcpyAsync(tmp, rotor_host, src_bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = launch_relayout(tmp, N, K, (*out)->tiles, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (tmp) (void)hipFree(tmp);
    if (e != hipSuccess) {
        rt_weights_free(*out);
        *out = nullptr;
        return hip_fail(e, "rt_weights_upload");
    }
    return RT_OK;
}

int rt_weights_download(rt_ctx* ctx, const rt_weights* w, uint8_t* rotor_host) {
    if (!ctx || !w || !rotor_host) return fail(RT_EINVAL, "rt_weights_download: NULL argument");
    DeviceGuard g(ctx->device);
    const size_t bytes = (size_t)w->N * ((w->K + 3) / 4);
    uint8_t* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, bytes);
    if (e == hipSuccess) e = launch_unrelayout(w->tiles, w->N, w->K, tmp, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(rotor_host, tmp, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (tmp) (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(e, "rt_weights_download");
    return RT_OK;
}

int rt_weights_info(const rt_weights* w, int* N, int* K, float* scale) {
    if (!w) return fail(RT_EINVAL, "rt_weights_info: w is NULL");
    if (N) *N = w->N;
    if (K) *K = w->K;
    if (scale) *scale = w->scale;
    return RT_OK;
}

int rt_weights_free(rt_weights* w) {
    if (!w) return RT_OK;
    DeviceGuard g(w->device);
    (void)hipDeviceSynchronize();  // launches still enqueued may read the tiles
    if (w->tiles) (void)hipFree(w->tiles);
    delete w;
    return RT_OK;
}

// --- activations -----------------------------------------------------------------

static int check_act(const rt_ctx* ctx, int M, int K, const char* who) {
    if (!ctx) return fail(RT_EINVAL, std::string(who) + ": ctx is NULL");
    if (M <= 0 || K <= 0) return fail(RT_EINVAL, std::string(who) + ": M and K must be positive");
    if (M > (1 << 24)) return fail(RT_EINVAL, std::string(who) + ": M too large");
    return RT_OK;
}

// Quantise (x != NULL) or permute (q_in != NULL) M rows of K into the context scratch.
static int stage_activations(rt_ctx* ctx, const float* x, const int8_t* q_in, int M, int K, int Mpad, bool blocked,
                             int8_t* q_nat, float* s_out, int8_t** qx, float** sx) {
    const int Kp = round_up(K, kChunk);
    const size_t qbytes = (size_t)Mpad * Kp;
    RT_HIP(ctx->act.ensure(qbytes + (size_t)Mpad * sizeof(float)));
    *qx = static_cast<int8_t*>(ctx->act.p);
    *sx = reinterpret_cast<float*>(static_cast<char*>(ctx->act.p) + qbytes);
    QuantArgs a{};
    a.dev = nullptr;
    a.U = 1;
    a.M = M;
    a.Mpad = Mpad;
    a.p = QuantProb{x, q_in, *qx, *sx, q_nat, K, Kp, q_in ? kPermute : kQuant, nullptr, 0.0f, nullptr, nullptr, 0, 0,
                    blocked};
    RT_HIP(launch_quant(a, ctx->stream, quant_rows_ok(a.p) ? K : 0));
    if (s_out) RT_HIP(hipMemcpyAsync(s_out, *sx, (size_t)M * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
    return RT_OK;
}

int rt_quantize_rows(rt_ctx* ctx, const float* x, int M, int K, int8_t* q, float* s) {
    int rc = check_act(ctx, M, K, "rt_quantize_rows");
    if (rc) return rc;
    if (!x || !q || !s) return fail(RT_EINVAL, "rt_quantize_rows: NULL pointer");
    DeviceGuard g(ctx->device);
    int8_t* qx;
    float* sx;
    return stage_activations(ctx, x, nullptr, M, K, M, false, q, s, &qx, &sx);
}

// M = 1 over fp32 inputs: can the quantisation run in the GEMV's prologue?  Sets
// a->has_pro / a->pro and *shape; false when the launch needs a separate quantiser pass.
// KSPLIT (few row blocks): only with one input shared by all problems.  ROWS: each
// workgroup quantises its own problem's row, so nw (4, 2 or 1 waves) must divide every
// problem's row-block count.
static bool prologue_launch(const GemvShape& base, int U, const int* Nb, int G, int Kp_max, const QuantProb& shared,
                            GemvArgs* a, GemvShape* shape) {
    const size_t row_lds = (size_t)Kp_max + sizeof(RowSmem);
    if (base.ksplit) {
        if (U != 1 || (size_t)base.nw * kRowBlock * sizeof(int) + row_lds > 64 * 1024) return false;
        a->has_pro = 1;
        a->pro = shared;
        *shape = base;
        return true;
    }
    if (row_lds > 64 * 1024) return false;
    int nw = 4;
    for (int g = 0; g < G; ++g)
        while (Nb[g] % nw) nw >>= 1;
    a->has_pro = 2;
    a->pro = QuantProb{};
    a->pro.Kp = Kp_max;
    *shape = GemvShape{false, nw};
    return true;
}

// GEMV (M <= kGemvMaxM) or MFMA GEMM on activations already in the qx layout.
static int launch_matrix(rt_ctx* ctx, const rt_weights* w, const int8_t* qx, const float* sx, int M,
                         const float* row_scale, void* out, bool out_i32, const float* res = nullptr) {
    if (M > kGemvMaxM) {
        if (!gemm_ldo_ok(M, w->N)) return fail(RT_EINVAL, "N too large for the GEMM's 32-bit output offsets at this M");
        GemmArgs a{w->tiles, qx, sx, row_scale, out, w->scale, M, w->N, w->Np, w->C, w->N, out_i32 ? 1 : 0, res};
        RT_HIP(launch_gemm(a, ctx->stream));
        return RT_OK;
    }
    const int mt = gemv_mt(M);
    GemvArgs a{};
    a.dev = nullptr;
    a.rb2p = nullptr;
    a.G = 1;
    a.M = M;
    a.out_i32 = out_i32 ? 1 : 0;
    a.total_rb = w->Np / kRowBlock;
    a.p = GemvProb{w->tiles, qx, sx, row_scale, out, w->scale, w->N, w->C, w->N, 0, res};
    const GemvShape shape = gemv_shape(a.total_rb, (M + mt - 1) / mt, w->C);
    RT_HIP(launch_gemv(a, mt, shape, ctx->stream));
    return RT_OK;
}

// M = 1 over fp32 x: ONE launch whose GEMV quantises x in its prologue, when the row fits
// the prologue's LDS (*launched = false otherwise; nothing is enqueued then).
static int linear_m1_prologue(rt_ctx* ctx, const rt_weights* w, const float* x, const float* row_scale, void* out,
                              bool* launched) {
    GemvArgs a{};
    a.G = 1;
    a.M = 1;
    a.total_rb = w->Np / kRowBlock;
    a.p = GemvProb{w->tiles, nullptr, nullptr, row_scale, out, w->scale, w->N, w->C, w->N, 0, nullptr, x, w->K};
    const QuantProb src{x, nullptr, nullptr, nullptr, nullptr, w->K, w->Kp, kQuant, nullptr, 0.0f, nullptr,
                        nullptr, 0, 0, 0};
    const int nb = a.total_rb;
    GemvShape shape;
    *launched = false;
    if (!prologue_launch(gemv_shape(a.total_rb, 1, w->C), 1, &nb, 1, w->Kp, src, &a, &shape)) return RT_OK;
    RT_HIP(launch_gemv(a, 1, shape, ctx->stream));
    *launched = true;
    return RT_OK;
}

static int run_linear(rt_ctx* ctx, const rt_weights* w, const float* x, const int8_t* q, int M,
                      const float* row_scale, void* out, bool out_i32, const char* who) {
    if (!w) return fail(RT_EINVAL, std::string(who) + ": weights are NULL");
    int rc = check_act(ctx, M, w->K, who);
    if (rc) return rc;
    if ((!x && !q) || !out) return fail(RT_EINVAL, std::string(who) + ": NULL pointer");
    if (w->device != ctx->device) return fail(RT_EINVAL, std::string(who) + ": weights live on another device");
    DeviceGuard g(ctx->device);
    if (M == 1 && x && !out_i32) {  // one launch: the GEMV quantises x in its prologue
        bool launched = false;
        rc = linear_m1_prologue(ctx, w, x, row_scale, out, &launched);
        if (rc || launched) return rc;
    }
    int8_t* qx;
    float* sx;
    rc = stage_activations(ctx, x, q, M, w->K, act_rows(M), qx_blocked(M), nullptr, nullptr, &qx, &sx);
    if (rc) return rc;
    return launch_matrix(ctx, w, qx, sx, M, row_scale, out, out_i32);
}

int rt_linear_i32(rt_ctx* ctx, const rt_weights* w, const int8_t* q, int M, int32_t* acc) {
    if (!q) return fail(RT_EINVAL, "rt_linear_i32: q is NULL");
    return run_linear(ctx, w, nullptr, q, M, nullptr, acc, true, "rt_linear_i32");
}

int rt_linear_f32(rt_ctx* ctx, const rt_weights* w, const float* x, int M, float* y) {
    if (!x) return fail(RT_EINVAL, "rt_linear_f32: x is NULL");
    return run_linear(ctx, w, x, nullptr, M, nullptr, y, false, "rt_linear_f32");
}

int rt_linear_f32_noalloc(rt_ctx* ctx, const rt_weights* w, const float* x, int M, float* y) {
    const char* who = "rt_linear_f32_noalloc";
    if (!w) return fail(RT_EINVAL, std::string(who) + ": weights are NULL");
    int rc = check_act(ctx, M, w->K, who);
    if (rc) return rc;
    if (!x || !y) return fail(RT_EINVAL, std::string(who) + ": NULL pointer");
    if (w->device != ctx->device) return fail(RT_EINVAL, std::string(who) + ": weights live on another device");
    if (!ctx->noalloc) return fail(RT_EINVAL, std::string(who) + ": the context has no static scratch");
    DeviceGuard g(ctx->device);
    if (M == 1) {
        bool launched = false;
        rc = linear_m1_prologue(ctx, w, x, nullptr, y, &launched);
        if (rc || launched) return rc;
    }
    // the activations of the GEMV / GEMM tile rows: int8 [Mpad][Kp], then fp32 scales [Mpad];
    // the quantiser writes every byte of both (padding rows as zeros), so what an earlier call
    // left in the buffer is never read
    const int Mpad = act_rows(M);
    const size_t qbytes = (size_t)Mpad * w->Kp, need = qbytes + (size_t)Mpad * sizeof(float);
    if (need > RT_NOALLOC_SCRATCH_BYTES)
        return fail(RT_EINVAL, std::string(who) + ": M = " + std::to_string(M) + ", K = " + std::to_string(w->K) +
                                   " needs " + std::to_string(need) + " bytes of activation scratch, more than the " +
                                   std::to_string(RT_NOALLOC_SCRATCH_BYTES) + " of the static buffer");
    int8_t* qx = ctx->noalloc;
    float* sx = reinterpret_cast<float*>(ctx->noalloc + qbytes);
    QuantArgs a{};
    a.U = 1;
    a.M = M;
    a.Mpad = Mpad;
    a.p = QuantProb{x, nullptr, qx, sx, nullptr, w->K, w->Kp, kQuant, nullptr, 0.0f, nullptr, nullptr, 0, 0,
                    qx_blocked(M)};
    RT_HIP(launch_quant(a, ctx->stream, quant_rows_ok(a.p) ? w->K : 0));
    return launch_matrix(ctx, w, qx, sx, M, nullptr, y, false);
}

int rt_linear_f32_rowscale(rt_ctx* ctx, const rt_weights* w, const float* x, int M, const float* row_scale,
                           float* y) {
    if (!x || !row_scale) return fail(RT_EINVAL, "rt_linear_f32_rowscale: NULL pointer");
    return run_linear(ctx, w, x, nullptr, M, row_scale, y, false, "rt_linear_f32_rowscale");
}

// --- plans -----------------------------------------------------------------------

int rt_plan_free(rt_plan* plan) {
    if (!plan) return RT_OK;
    DeviceGuard g(plan->device);
    (void)hipDeviceSynchronize();  // launches still enqueued may read the descriptors
    if (plan->dev_probs) (void)hipFree(plan->dev_probs);
    if (plan->dev_rb2p) (void)hipFree(plan->dev_rb2p);
    if (plan->dev_gemms) (void)hipFree(plan->dev_gemms);
    if (plan->dev_tile2p) (void)hipFree(plan->dev_tile2p);
    if (plan->dev_unit2d) (void)hipFree(plan->dev_unit2d);
    if (plan->gemm_cnt) (void)hipFree(plan->gemm_cnt);
    if (plan->gemm_ws) (void)hipFree(plan->gemm_ws);
    if (plan->dev_quant) (void)hipFree(plan->dev_quant);
    if (plan->act) (void)hipFree(plan->act);
    if (plan->att_mem) (void)hipFree(plan->att_mem);
    delete plan;
    return RT_OK;
}

// M > 8: one launch serves all problems.  M <= 64: the split-K kernel, one unit per row
// block and part (upload_splitk_group).  M > 64: the tile kernel, the tiles of problem g
// after those of problems 0..g-1, with a tile -> problem table.
// Split-K parts of a problem with C chunks when the group's shortest problem has Cmin: a
// problem several times longer than the shortest is cut into about C / Cmin parts (at most
// 8), so that no workgroup walks far more chunks than the others.
static int splitk_parts(int C, int Cmin) { return std::max(1, std::min(8, (C + Cmin / 2) / std::max(Cmin, 1))); }

// the bounds a grouped GEMM launch passes in its arguments (-1: too many descriptors, the
// launch reads its unit -> descriptor table instead)
static int group_bounds(const rt_plan* p) {
    return (int)p->gemm_bnd.size() <= kGroupBounds ? (int)p->gemm_bnd.size() : -1;
}

static hipError_t upload_splitk_group(rt_plan* p) {
    const std::vector<GemmArgs>& g = p->gemms;
    int Cmin = 1 << 30;
    for (const GemmArgs& a : g) Cmin = std::min(Cmin, a.C);
    std::vector<GemmArgs> d;  // descriptors: every part of every problem
    std::vector<int> unit2d;
    size_t cnt_n = 0, ws_n = 0;
    std::vector<std::pair<size_t, size_t>> offs(g.size());  // counter, workspace offsets of split problems
    for (size_t i = 0; i < g.size(); ++i) {
        const int parts = splitk_parts(g[i].C, Cmin), nrb = g[i].Np / kRowBlock;
        offs[i] = {cnt_n, ws_n};
        if (parts > 1) {
            cnt_n += (size_t)nrb;
            ws_n += (size_t)parts * nrb * 4096;
        }
    }
    hipError_t e = hipSuccess;
    if (cnt_n) {
        e = hipMalloc(&p->gemm_cnt, cnt_n * sizeof(int));
        if (e == hipSuccess) e = hipMemset(p->gemm_cnt, 0, cnt_n * sizeof(int));
        if (e == hipSuccess) e = hipMalloc(&p->gemm_ws, ws_n * sizeof(int));
        if (e != hipSuccess) return e;
    }
    // the split problems' workgroups first in the grid: they walk their part of K and then
    // hand over, so starting them first shortens the launch
    std::vector<size_t> order;
    for (int pass = 0; pass < 2; ++pass)
        for (size_t i = 0; i < g.size(); ++i)
            if ((splitk_parts(g[i].C, Cmin) > 1) == (pass == 0)) order.push_back(i);
    for (size_t i : order) {
        const int parts = splitk_parts(g[i].C, Cmin), nrb = g[i].Np / kRowBlock;
        for (int kp = 0; kp < parts; ++kp) {
            GemmArgs a = g[i];
            a.wg_begin = (int)unit2d.size();
            a.kp = kp;
            a.parts = parts;
            a.c0 = (int)((long long)kp * a.C / parts);
            a.c1 = (int)((long long)(kp + 1) * a.C / parts);
            a.cnt = parts > 1 ? p->gemm_cnt + offs[i].first : nullptr;
            a.part_ws = parts > 1 ? p->gemm_ws + offs[i].second : nullptr;
            if (!d.empty()) p->gemm_bnd.push_back((int)unit2d.size());
            unit2d.insert(unit2d.end(), (size_t)nrb, (int)d.size());
            d.push_back(a);
        }
    }
    if (unit2d.empty() || unit2d.size() > (1u << 30)) return hipErrorInvalidValue;
    p->gemm_units = (int)unit2d.size();
    e = hipMalloc(&p->dev_gemms, sizeof(GemmArgs) * d.size());
    if (e == hipSuccess) e = hipMemcpy(p->dev_gemms, d.data(), sizeof(GemmArgs) * d.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc(&p->dev_unit2d, sizeof(int) * unit2d.size());
    if (e == hipSuccess)
        e = hipMemcpy(p->dev_unit2d, unit2d.data(), sizeof(int) * unit2d.size(), hipMemcpyHostToDevice);
    return e;
}

static hipError_t upload_gemm_group(rt_plan* p) {
    if (p->gemms.empty()) return hipSuccess;
    if (gemm_bm(p->M) == 64) return upload_splitk_group(p);
    std::vector<GemmArgs> g = p->gemms;
    std::vector<int> tile2p;
    std::vector<int> Ns(g.size()), Cs(g.size());
    for (size_t i = 0; i < g.size(); ++i) {
        Ns[i] = g[i].N;
        Cs[i] = g[i].C;
    }
    p->gemm_cfg = gemm_tile_cfg(p->M, Ns.data(), Cs.data(), (int)g.size());
    // the pair epilogue runs in tiles whose waves hold one 64-column group: not the 64-row
    // tile's 32 columns, the 256-column tile's 128 or the region kernel (its own epilogue)
    if (p->pair_gemm && (p->gemm_cfg == kTile64x128 || p->gemm_cfg == kRegion128x160)) p->gemm_cfg = kTile128x128;
    if (p->pair_gemm && p->gemm_cfg == kTile256x256) p->gemm_cfg = kTile256x128;
    long long total = 0;
    for (size_t i = 0; i < g.size(); ++i) {
        g[i].wg_begin = (int)total;
        if (i > 0) p->gemm_bnd.push_back((int)total);
        const long long n = gemm_tile_count(p->gemm_cfg, p->M, g[i].N);
        tile2p.insert(tile2p.end(), (size_t)n, (int)i);
        total += n;
    }
    if (total <= 0 || total > (1 << 30)) return hipErrorInvalidValue;
    p->gemm_tiles = (int)total;
    hipError_t e = hipMalloc(&p->dev_gemms, sizeof(GemmArgs) * g.size());
    if (e == hipSuccess) e = hipMemcpy(p->dev_gemms, g.data(), sizeof(GemmArgs) * g.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && !tile2p.empty()) {
        e = hipMalloc(&p->dev_tile2p, sizeof(int) * tile2p.size());
        if (e == hipSuccess)
            e = hipMemcpy(p->dev_tile2p, tile2p.data(), sizeof(int) * tile2p.size(), hipMemcpyHostToDevice);
    }
    return e;
}

int rt_plan_create(rt_ctx* ctx, int G, const rt_weights* const* w, const float* const* x, int M, float* const* y,
                   rt_plan** out) {
    if (!ctx || !w || !x || !y || !out) return fail(RT_EINVAL, "rt_plan_create: NULL argument");
    *out = nullptr;
    if (G <= 0 || G > (1 << 16)) return fail(RT_EINVAL, "rt_plan_create: G out of range");
    if (M <= 0 || M > (1 << 24)) return fail(RT_EINVAL, "rt_plan_create: M out of range");
    for (int g = 0; g < G; ++g) {
        if (!w[g] || !x[g] || !y[g]) return fail(RT_EINVAL, "rt_plan_create: NULL entry in a pointer array");
        if (w[g]->device != ctx->device) return fail(RT_EINVAL, "rt_plan_create: weights live on another device");
        if (M > kGemvMaxM && !gemm_ldo_ok(M, w[g]->N))
            return fail(RT_EINVAL, "rt_plan_create: N too large for the GEMM's 32-bit output offsets at this M");
    }
    DeviceGuard guard(ctx->device);
    rt_plan* p = new rt_plan();
    p->device = ctx->device;
    p->G = G;
    p->M = M;
    p->mt = gemv_mt(M);
    p->Mpad = M > kGemvMaxM ? round_up(M, gemm_bm(M)) : round_up(M, p->mt);
    // distinct inputs (same pointer => same quantisation; their K must agree)
    std::unordered_map<const float*, int> uid;
    std::vector<int> which(G);
    std::vector<int> Ku;
    for (int g = 0; g < G; ++g) {
        auto it = uid.find(x[g]);
        if (it == uid.end()) {
            which[g] = (int)Ku.size();
            uid.emplace(x[g], which[g]);
            Ku.push_back(w[g]->K);
        } else {
            which[g] = it->second;
            if (Ku[it->second] != w[g]->K) {
                delete p;
                return fail(RT_EINVAL, "rt_plan_create: problems sharing an input have different K");
            }
        }
    }
    p->U = (int)Ku.size();
    std::vector<size_t> qoff(p->U), soff(p->U);
    size_t total = 0;
    for (int u = 0; u < p->U; ++u) {
        qoff[u] = total;
        total += (size_t)p->Mpad * round_up(Ku[u], kChunk);
        total = (total + 255) / 256 * 256;
    }
    for (int u = 0; u < p->U; ++u) {
        soff[u] = total;
        total += (size_t)p->Mpad * sizeof(float);
        total = (total + 255) / 256 * 256;
    }
    hipError_t e = hipMalloc(&p->act, total);
    if (e != hipSuccess) {
        delete p;
        return fail(RT_ENOMEM, "rt_plan_create: activation buffer allocation failed");
    }
    char* base = static_cast<char*>(p->act);
    p->quant.resize(p->U);
    for (int g = 0; g < G; ++g) {
        const int u = which[g];
        p->quant[u] = QuantProb{x[g], nullptr, reinterpret_cast<int8_t*>(base + qoff[u]),
                                reinterpret_cast<float*>(base + soff[u]), nullptr, Ku[u], round_up(Ku[u], kChunk),
                                kQuant, nullptr, 0.0f, nullptr, nullptr, 0, 0, qx_blocked(M)};
    }
    p->quant_maxK = 0;
    for (const QuantProb& qp : p->quant) {
        if (!quant_rows_ok(qp)) {
            p->quant_maxK = 0;
            break;
        }
        p->quant_maxK = std::max(p->quant_maxK, qp.K);
    }
    int wg = 0, minC = 1 << 30;
    p->probs.resize(G);
    for (int g = 0; g < G; ++g) {
        const int u = which[g];
        p->probs[g] = GemvProb{w[g]->tiles, p->quant[u].qx, p->quant[u].sx, nullptr, y[g], w[g]->scale,
                               w[g]->N, w[g]->C, w[g]->N, wg};
        wg += w[g]->Np / kRowBlock;
        if (w[g]->C < minC) minC = w[g]->C;
    }
    p->total_rb = wg;
    p->shape = gemv_shape(wg, (M + p->mt - 1) / p->mt, minC);
    if (M == 1) {
        std::vector<int> nb(G);
        int kp_max = 0;
        for (int g = 0; g < G; ++g) {
            p->probs[g].xs = x[g];
            p->probs[g].K = w[g]->K;
            nb[g] = w[g]->Np / kRowBlock;
            kp_max = std::max(kp_max, round_up(w[g]->K, kChunk));
        }
        GemvArgs probe{};
        if (prologue_launch(p->shape, p->U, nb.data(), G, kp_max, p->quant[0], &probe, &p->run_shape)) {
            p->run_pro = probe.has_pro;
            p->pro = probe.pro;
        }
    }
    if (M > kGemvMaxM)
        for (int g = 0; g < G; ++g)
            p->gemms.push_back(GemmArgs{w[g]->tiles, p->probs[g].qx, p->probs[g].sx, nullptr, y[g], w[g]->scale, M,
                                        w[g]->N, w[g]->Np, w[g]->C, w[g]->N, 0});
    std::vector<int> rb2p(wg);
    for (int g = 0; g < G; ++g)
        for (int r = 0; r < w[g]->Np / kRowBlock; ++r) rb2p[p->probs[g].wg_begin + r] = g;
    e = hipMalloc(&p->dev_probs, sizeof(GemvProb) * G);
    if (e == hipSuccess) e = hipMalloc(&p->dev_rb2p, sizeof(int) * wg);
    if (e == hipSuccess) e = hipMemcpy(p->dev_rb2p, rb2p.data(), sizeof(int) * wg, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc(&p->dev_quant, sizeof(QuantProb) * p->U);
    if (e == hipSuccess)
        e = hipMemcpy(p->dev_probs, p->probs.data(), sizeof(GemvProb) * G, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(p->dev_quant, p->quant.data(), sizeof(QuantProb) * p->U, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = upload_gemm_group(p);
    if (e != hipSuccess) {
        rt_plan_free(p);
        return hip_fail(e, "rt_plan_create");
    }
    *out = p;
    return RT_OK;
}

int rt_plan_describe(const rt_plan* plan, int* kind, int* tile_m, int* tile_n, int* units) {
    if (!plan) return fail(RT_EINVAL, "rt_plan_describe: plan is NULL");
    int k, tm, tn, u;
    if (plan->dev_tile2p) {
        k = RT_LAUNCH_TILES;
        tm = gemm_tile_bm(plan->gemm_cfg);
        tn = gemm_tile_bn(plan->gemm_cfg);
        u = plan->gemm_tiles;
    } else if (plan->dev_gemms) {
        k = RT_LAUNCH_SPLITK;
        tm = 64;
        tn = kRowBlock;
        u = plan->gemm_units;
    } else if (plan->fused || plan->run_pro) {
        k = RT_LAUNCH_GEMV_FUSED;
        const GemvShape sh = plan->fused ? plan->shape : plan->run_shape;
        tm = 1;
        tn = sh.ksplit ? kRowBlock : kRowBlock * sh.nw;
        u = sh.ksplit ? plan->total_rb : plan->total_rb / sh.nw;
    } else {
        k = RT_LAUNCH_GEMV;
        tm = plan->mt;
        tn = plan->shape.ksplit ? kRowBlock : kRowBlock * plan->shape.nw;
        u = (plan->shape.ksplit ? plan->total_rb : (plan->total_rb + plan->shape.nw - 1) / plan->shape.nw) *
            ((plan->M + plan->mt - 1) / plan->mt);
    }
    if (kind) *kind = k;
    if (tile_m) *tile_m = tm;
    if (tile_n) *tile_n = tn;
    if (units) *units = u;
    return RT_OK;
}

// Plans of up to kInlineProbs problems pass their descriptors as kernel arguments.
// (launch_gemv fills the leading weight-stream table from them.)
static void inline_probs(const rt_plan* plan, GemvArgs* a) {
    if (plan->G > kInlineProbs) return;
    a->ninl = plan->G;
    for (int g = 0; g < plan->G; ++g) a->inl[g] = plan->probs[g];
}

int rt_plan_quantize(rt_ctx* ctx, const rt_plan* plan) {
    if (!ctx || !plan) return fail(RT_EINVAL, "rt_plan_quantize: NULL argument");
    if (plan->device != ctx->device) return fail(RT_EINVAL, "rt_plan_quantize: plan belongs to another device");
    DeviceGuard g(ctx->device);
    QuantArgs q{};
    q.dev = plan->dev_quant;
    q.U = plan->U;
    q.M = plan->M;
    q.Mpad = plan->Mpad;
    RT_HIP(launch_quant(q, ctx->stream, plan->quant_maxK));
    return RT_OK;
}

int rt_plan_run(rt_ctx* ctx, const rt_plan* plan) {
    if (plan && plan->run_pro && ctx && plan->device == ctx->device) {  // one launch: quantise in the prologue
        DeviceGuard g(ctx->device);
        GemvArgs a{};
        a.dev = plan->dev_probs;
        a.rb2p = plan->dev_rb2p;
        inline_probs(plan, &a);
        a.G = plan->G;
        a.M = 1;
        a.out_i32 = 0;
        a.total_rb = plan->total_rb;
        a.has_pro = plan->run_pro;
        a.pro = plan->pro;
        RT_HIP(launch_gemv(a, 1, plan->run_shape, ctx->stream));
        return RT_OK;
    }
    int rc = rt_plan_quantize(ctx, plan);
    return rc ? rc : rt_plan_gemv(ctx, plan);
}

int rt_plan_gemv(rt_ctx* ctx, const rt_plan* plan) {
    if (!ctx || !plan) return fail(RT_EINVAL, "rt_plan_gemv: NULL argument");
    if (plan->device != ctx->device) return fail(RT_EINVAL, "rt_plan_gemv: plan belongs to another device");
    for (const rt_act* act : plan->acts)
        if (act->M != plan->M) return fail(RT_EINVAL, "rt_plan_gemv: an input activation does not hold the plan's M tokens");
    DeviceGuard g(ctx->device);
    GemvArgs a{};
    if (plan->fused) {
        a.has_pro = 1;
        a.pro = plan->pro;
        a.pair_a = plan->pair_a;
        a.pair_ssq = plan->pair_ssq;
        a.out_ssq = plan->out_ssq;
        a.pair_g = plan->pair_g;
        a.pair_u = plan->pair_u;
        a.pair_sg = plan->pair_sg;
        a.pair_su = plan->pair_su;
    }
    a.dev = plan->dev_probs;
    a.rb2p = plan->dev_rb2p;
    inline_probs(plan, &a);
    a.G = plan->G;
    a.M = plan->M;
    a.out_i32 = 0;
    a.total_rb = plan->total_rb;
    if (plan->dev_tile2p) {
        RT_HIP(launch_gemm_tiles(plan->dev_gemms, plan->dev_tile2p, plan->gemm_bnd.data(), group_bounds(plan),
                                 plan->gemm_tiles, plan->gemm_cfg, ctx->stream));
        return RT_OK;
    }
    if (plan->dev_gemms) {
        RT_HIP(launch_gemm_group(plan->dev_gemms, plan->dev_unit2d, plan->gemm_bnd.data(), group_bounds(plan),
                                 plan->gemm_units, ctx->stream));
        return RT_OK;
    }
    if (plan->att_on)
        RT_HIP(launch_gemv_attn(a, plan->att, plan->att_Hkv, plan->att_hd, plan->shape, ctx->stream));
    else
        RT_HIP(launch_gemv(a, plan->mt, plan->shape, ctx->stream));
    return RT_OK;
}

// --- reusable quantised activations ------------------------------------------------

int rt_act_create(rt_ctx* ctx, int M, int K, rt_act** out) {
    if (!ctx || !out) return fail(RT_EINVAL, "rt_act_create: NULL argument");
    *out = nullptr;
    if (M <= 0 || K <= 0 || M > (1 << 24) || K > (1 << 24)) return fail(RT_EINVAL, "rt_act_create: M or K out of range");
    DeviceGuard g(ctx->device);
    rt_act* a = new rt_act();
    a->device = ctx->device;
    a->Mcap = M;
    a->K = K;
    a->Kp = round_up(K, kChunk);
    a->Mpad_cap = act_rows(M);
    for (int m = 1; m <= M; ++m) a->Mpad_cap = std::max(a->Mpad_cap, act_rows(m));
    const size_t qbytes = (size_t)a->Mpad_cap * a->Kp;
    hipError_t e = hipMalloc(&a->mem, qbytes + (size_t)a->Mpad_cap * sizeof(float));
    if (e != hipSuccess) {
        delete a;
        return fail(RT_ENOMEM, "rt_act_create: allocation failed");
    }
    a->qx = static_cast<int8_t*>(a->mem);
    a->sx = reinterpret_cast<float*>(static_cast<char*>(a->mem) + qbytes);
    *out = a;
    return RT_OK;
}

int rt_act_free(rt_act* act) {
    if (!act) return RT_OK;
    DeviceGuard g(act->device);
    (void)hipDeviceSynchronize();  // launches still enqueued may read the activations
    if (act->mem) (void)hipFree(act->mem);
    delete act;
    return RT_OK;
}

static int act_fill(rt_ctx* ctx, rt_act* act, int M, int mode, const float* x, const float* aux, float eps,
                    float* v_out, const char* who, const float* aux2 = nullptr) {
    if (!ctx || !act || !x) return fail(RT_EINVAL, std::string(who) + ": NULL argument");
    if (M <= 0 || M > act->Mcap) return fail(RT_EINVAL, std::string(who) + ": M exceeds the activation capacity");
    if (act->device != ctx->device) return fail(RT_EINVAL, std::string(who) + ": activations live on another device");
    DeviceGuard g(ctx->device);
    QuantArgs q{};
    q.dev = nullptr;
    q.U = 1;
    q.M = M;
    q.Mpad = act_rows(M);
    q.p = QuantProb{x, nullptr, act->qx, act->sx, nullptr, act->K, act->Kp, mode, aux, eps, v_out, aux2, 0, 0,
                    qx_blocked(M)};
    RT_HIP(launch_quant(q, ctx->stream, quant_rows_ok(q.p) ? act->K : 0));
    act->M = M;
    act->Mpad = q.Mpad;
    return RT_OK;
}

int rt_act_quantize(rt_ctx* ctx, const float* x, int M, rt_act* act) {
    return act_fill(ctx, act, M, kQuant, x, nullptr, 0.0f, nullptr, "rt_act_quantize");
}

int rt_act_rmsnorm_quantize(rt_ctx* ctx, const float* x, const float* norm_w, float eps, int M, rt_act* act,
                            float* h_out) {
    if (!norm_w) return fail(RT_EINVAL, "rt_act_rmsnorm_quantize: norm weight is NULL");
    return act_fill(ctx, act, M, kRmsNorm, x, norm_w, eps, h_out, "rt_act_rmsnorm_quantize");
}

int rt_act_relu2_mul_quantize(rt_ctx* ctx, const float* gate, const float* up, int M, rt_act* act, float* a_out) {
    if (!up) return fail(RT_EINVAL, "rt_act_relu2_mul_quantize: up is NULL");
    return act_fill(ctx, act, M, kRelu2Mul, gate, up, 0.0f, a_out, "rt_act_relu2_mul_quantize");
}

int rt_act_relu2_mul_norm_quantize(rt_ctx* ctx, const float* gate, const float* up, const float* norm_w, float eps,
                                   int M, rt_act* act, float* a_out) {
    if (!up || !norm_w) return fail(RT_EINVAL, "rt_act_relu2_mul_norm_quantize: NULL argument");
    return act_fill(ctx, act, M, kRelu2MulNorm, gate, up, eps, a_out, "rt_act_relu2_mul_norm_quantize", norm_w);
}

int rt_act_export(rt_ctx* ctx, const rt_act* act, int8_t* q, float* s) {
    if (!ctx || !act || !q || !s) return fail(RT_EINVAL, "rt_act_export: NULL argument");
    if (act->M <= 0) return fail(RT_EINVAL, "rt_act_export: activations are empty");
    DeviceGuard g(ctx->device);
    RT_HIP(launch_unpermute(act->qx, act->M, act->K, act->Kp, qx_blocked(act->M), q, ctx->stream));
    RT_HIP(hipMemcpyAsync(s, act->sx, (size_t)act->M * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
    return RT_OK;
}

int rt_linear_act_f32(rt_ctx* ctx, const rt_weights* w, const rt_act* act, const float* residual, float* y) {
    if (!ctx || !w || !act || !y) return fail(RT_EINVAL, "rt_linear_act_f32: NULL argument");
    if (act->M <= 0) return fail(RT_EINVAL, "rt_linear_act_f32: activations are empty");
    if (act->K != w->K) return fail(RT_EINVAL, "rt_linear_act_f32: activation K differs from the weights' K");
    if (w->device != ctx->device || act->device != ctx->device)
        return fail(RT_EINVAL, "rt_linear_act_f32: operands live on another device");
    DeviceGuard g(ctx->device);
    return launch_matrix(ctx, w, act->qx, act->sx, act->M, nullptr, y, false, residual);
}

int rt_plan_create_act(rt_ctx* ctx, int G, const rt_weights* const* w, const rt_act* const* act, int M,
                       float* const* y, rt_plan** out) {
    if (!ctx || !w || !act || !y || !out) return fail(RT_EINVAL, "rt_plan_create_act: NULL argument");
    *out = nullptr;
    if (G <= 0 || G > (1 << 16)) return fail(RT_EINVAL, "rt_plan_create_act: G out of range");
    for (int g = 0; g < G; ++g) {
        if (!w[g] || !act[g] || !y[g]) return fail(RT_EINVAL, "rt_plan_create_act: NULL entry in a pointer array");
        if (act[g]->K != w[g]->K) return fail(RT_EINVAL, "rt_plan_create_act: activation K differs from weights");
        if (M <= 0 || M > act[g]->Mcap) return fail(RT_EINVAL, "rt_plan_create_act: M exceeds an activation capacity");
        if (w[g]->device != ctx->device || act[g]->device != ctx->device)
            return fail(RT_EINVAL, "rt_plan_create_act: operands live on another device");
        if (M > kGemvMaxM && !gemm_ldo_ok(M, w[g]->N))
            return fail(RT_EINVAL, "rt_plan_create_act: N too large for the GEMM's 32-bit output offsets at this M");
    }
    DeviceGuard guard(ctx->device);
    rt_plan* p = new rt_plan();
    p->device = ctx->device;
    p->G = G;
    p->M = M;
    p->mt = gemv_mt(M);
    p->Mpad = act_rows(M);
    p->U = 0;  // inputs are quantised by the caller
    p->acts.assign(act, act + G);
    int wg = 0, minC = 1 << 30;
    p->probs.resize(G);
    for (int g = 0; g < G; ++g) {
        p->probs[g] = GemvProb{w[g]->tiles, act[g]->qx, act[g]->sx, nullptr, y[g], w[g]->scale,
                               w[g]->N, w[g]->C, w[g]->N, wg};
        wg += w[g]->Np / kRowBlock;
        if (w[g]->C < minC) minC = w[g]->C;
        if (M > kGemvMaxM)
            p->gemms.push_back(GemmArgs{w[g]->tiles, act[g]->qx, act[g]->sx, nullptr, y[g], w[g]->scale, M,
                                        w[g]->N, w[g]->Np, w[g]->C, w[g]->N, 0});
    }
    p->total_rb = wg;
    p->shape = gemv_shape(wg, (M + p->mt - 1) / p->mt, minC);
    std::vector<int> rb2p(wg);
    for (int g = 0; g < G; ++g)
        for (int r = 0; r < w[g]->Np / kRowBlock; ++r) rb2p[p->probs[g].wg_begin + r] = g;
    hipError_t e = hipMalloc(&p->dev_probs, sizeof(GemvProb) * G);
    if (e == hipSuccess) e = hipMalloc(&p->dev_rb2p, sizeof(int) * wg);
    if (e == hipSuccess) e = hipMemcpy(p->dev_rb2p, rb2p.data(), sizeof(int) * wg, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p->dev_probs, p->probs.data(), sizeof(GemvProb) * G, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = upload_gemm_group(p);
    if (e != hipSuccess) {
        rt_plan_free(p);
        return hip_fail(e, "rt_plan_create_act");
    }
    *out = p;
    return RT_OK;
}

int rt_plan_create_act_gate_up(rt_ctx* ctx, const rt_weights* w_gu, float s_gate, float s_up, const rt_act* act,
                               int M, float* a_out, rt_plan** out) {
    const char* who = "rt_plan_create_act_gate_up";
    if (!ctx || !w_gu || !act || !a_out || !out) return fail(RT_EINVAL, std::string(who) + ": NULL argument");
    *out = nullptr;
    if (act->K != w_gu->K) return fail(RT_EINVAL, std::string(who) + ": activation K differs from weights");
    if (M <= 64 || M > act->Mcap)
        return fail(RT_EINVAL, std::string(who) + ": M must exceed 64 (the tile GEMM) and fit the activations");
    if (w_gu->N % 64) return fail(RT_EINVAL, std::string(who) + ": the interleaved matrix needs N % 64 == 0");
    if (w_gu->device != ctx->device || act->device != ctx->device)
        return fail(RT_EINVAL, std::string(who) + ": operands live on another device");
    if (!gemm_ldo_ok(M, w_gu->N)) return fail(RT_EINVAL, std::string(who) + ": N too large for 32-bit offsets");
    DeviceGuard guard(ctx->device);
    rt_plan* p = new rt_plan();
    p->device = ctx->device;
    p->G = 1;
    p->M = M;
    p->mt = gemv_mt(M);
    p->Mpad = act_rows(M);
    p->U = 0;  // the input is quantised by the caller
    p->acts.assign(1, act);
    p->pair_gemm = true;
    const int F = w_gu->N / 2;
    p->probs.assign(1, GemvProb{w_gu->tiles, act->qx, act->sx, nullptr, a_out, 1.0f, w_gu->N, w_gu->C, F, 0});
    p->total_rb = w_gu->Np / kRowBlock;
    GemmArgs ga{w_gu->tiles, act->qx, act->sx, nullptr, nullptr, 1.0f, M, w_gu->N, w_gu->Np, w_gu->C, F, 0};
    ga.pair_a = a_out;
    ga.pair_sg = s_gate;
    ga.pair_su = s_up;
    p->gemms.push_back(ga);
    hipError_t e = upload_gemm_group(p);
    if (e != hipSuccess) {
        rt_plan_free(p);
        return hip_fail(e, who);
    }
    *out = p;
    return RT_OK;
}

// --- model kernels --------------------------------------------------------------------

int rt_embed(rt_ctx* ctx, const uint16_t* emb, int V, int D, const int* ids, int M, float* h) {
    if (!ctx || !emb || !ids || !h) return fail(RT_EINVAL, "rt_embed: NULL argument");
    if (V <= 0 || D <= 0 || M <= 0) return fail(RT_EINVAL, "rt_embed: sizes must be positive");
    DeviceGuard g(ctx->device);
    RT_HIP(launch_embed(emb, ids, M, V, D, h, ctx->stream));
    return RT_OK;
}

static int check_heads(int H, int Hkv, int hd, int Lmax, const char* who) {
    if (H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || hd % 2 || 256 % hd || Lmax <= 0 || Lmax > (1 << 16))
        return fail(RT_EINVAL, std::string(who) + ": unsupported head layout (H % Hkv == 0, even hd dividing 256, "
                                                  "Lmax <= 65536)");
    return RT_OK;
}

int rt_rope_kv_append(rt_ctx* ctx, float* q, float* k, const float* v, float* k_cache, float* v_cache,
                      const float* rope, int M, int H, int Hkv, int hd, int Lmax, const int* pos) {
    if (!ctx || !q || !k || !v || !k_cache || !v_cache || !rope || !pos)
        return fail(RT_EINVAL, "rt_rope_kv_append: NULL argument");
    int rc = check_heads(H, Hkv, hd, Lmax, "rt_rope_kv_append");
    if (rc) return rc;
    if (M <= 0 || M > Lmax) return fail(RT_EINVAL, "rt_rope_kv_append: M out of range");
    DeviceGuard g(ctx->device);
    RT_HIP(launch_rope_append(q, k, v, k_cache, v_cache, rope, M, H, Hkv, hd, Lmax, pos, ctx->stream));
    return RT_OK;
}

int rt_attention(rt_ctx* ctx, const float* q, const float* k_cache, const float* v_cache, float* out, int M, int H,
                 int Hkv, int hd, int Lmax, const int* pos) {
    if (!ctx || !q || !k_cache || !v_cache || !out || !pos) return fail(RT_EINVAL, "rt_attention: NULL argument");
    int rc = check_heads(H, Hkv, hd, Lmax, "rt_attention");
    if (rc) return rc;
    if (M <= 0 || M > Lmax) return fail(RT_EINVAL, "rt_attention: M out of range");
    if ((size_t)(hd + Lmax + 256) * sizeof(float) > 160 * 1024)
        return fail(RT_EINVAL, "rt_attention: Lmax too large for the scores buffer");
    DeviceGuard g(ctx->device);
    RT_HIP(launch_attention(q, k_cache, v_cache, out, M, H, Hkv, hd, Lmax, pos, 1.0f / sqrtf((float)hd),
                            ctx->stream));
    return RT_OK;
}

size_t rt_attention_decode_workspace(int H, int hd, int Lmax) {
    return (size_t)H * attn_splits(Lmax) * (hd + 2) * sizeof(float);
}

static int attn_decode_check(rt_ctx* ctx, const float* q, const float* kc, const float* vc, const int* pos, void* ws,
                             size_t ws_bytes, int H, int Hkv, int hd, int Lmax, const char* who) {
    if (!ctx || !q || !kc || !vc || !pos || !ws) return fail(RT_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_heads(H, Hkv, hd, Lmax, who);
    if (rc) return rc;
    if (hd != 64 && hd != 128) return fail(RT_EINVAL, std::string(who) + ": head_dim must be 64 or 128");
    if (ws_bytes < rt_attention_decode_workspace(H, hd, Lmax))
        return fail(RT_EINVAL, std::string(who) + ": workspace too small");
    return RT_OK;
}

int rt_attention_decode_partials(rt_ctx* ctx, const float* q, const float* k_cache, const float* v_cache, int H,
                                 int Hkv, int hd, int Lmax, const int* pos, void* workspace, size_t workspace_bytes) {
    int rc = attn_decode_check(ctx, q, k_cache, v_cache, pos, workspace, workspace_bytes, H, Hkv, hd, Lmax,
                               "rt_attention_decode_partials");
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    RT_HIP(launch_attn_partial(q, nullptr, nullptr, const_cast<float*>(k_cache), const_cast<float*>(v_cache), nullptr,
                               H, Hkv, hd, Lmax, pos, 1.0f / sqrtf((float)hd), static_cast<float*>(workspace),
                               ctx->stream));
    return RT_OK;
}

int rt_rope_attention_decode(rt_ctx* ctx, const float* q, const float* k, const float* v, float* k_cache,
                             float* v_cache, const float* rope, int H, int Hkv, int hd, int Lmax, const int* pos,
                             void* workspace, size_t workspace_bytes, float* out) {
    int rc = attn_decode_check(ctx, q, k_cache, v_cache, pos, workspace, workspace_bytes, H, Hkv, hd, Lmax,
                               "rt_rope_attention_decode");
    if (rc) return rc;
    if (!k || !v || !rope) return fail(RT_EINVAL, "rt_rope_attention_decode: NULL argument");
    DeviceGuard g(ctx->device);
    RT_HIP(launch_attn_partial(q, k, v, k_cache, v_cache, rope, H, Hkv, hd, Lmax, pos, 1.0f / sqrtf((float)hd),
                               static_cast<float*>(workspace), ctx->stream));
    if (out)
        RT_HIP(launch_attn_combine(static_cast<const float*>(workspace), H, hd, attn_splits(Lmax), out, ctx->stream));
    return RT_OK;
}

int rt_attention_decode(rt_ctx* ctx, const float* q, const float* k_cache, const float* v_cache, float* out, int H,
                        int Hkv, int hd, int Lmax, const int* pos, void* workspace, size_t workspace_bytes) {
    if (!out) return fail(RT_EINVAL, "rt_attention_decode: out is NULL");
    int rc = rt_attention_decode_partials(ctx, q, k_cache, v_cache, H, Hkv, hd, Lmax, pos, workspace, workspace_bytes);
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    RT_HIP(launch_attn_combine(static_cast<const float*>(workspace), H, hd, attn_splits(Lmax), out, ctx->stream));
    return RT_OK;
}

int rt_attention_decode_combine(rt_ctx* ctx, const void* workspace, size_t workspace_bytes, int H, int hd, int Lmax,
                                float* out) {
    const char* who = "rt_attention_decode_combine";
    if (!ctx || !workspace || !out) return fail(RT_EINVAL, std::string(who) + ": NULL argument");
    if (H <= 0 || hd <= 0 || Lmax <= 0) return fail(RT_EINVAL, std::string(who) + ": H, hd and Lmax must be positive");
    if (workspace_bytes < rt_attention_decode_workspace(H, hd, Lmax))
        return fail(RT_EINVAL, std::string(who) + ": workspace too small");
    DeviceGuard g(ctx->device);
    RT_HIP(launch_attn_combine(static_cast<const float*>(workspace), H, hd, attn_splits(Lmax), out, ctx->stream));
    return RT_OK;
}

int rt_lm_head_argmax(rt_ctx* ctx, const uint16_t* emb, const float* x, const float* norm_w, float eps, int V, int D,
                      float* logits, unsigned long long* best, int* token, int* pos, int advance, int* next_ids,
                      int* out_tokens, int pos_base, int out_cap, float* next_h) {
    if (!ctx || !emb || !x || !norm_w || !logits || !best || !token)
        return fail(RT_EINVAL, "rt_lm_head_argmax: NULL argument");
    if (V <= 0 || D <= 0 || D % 512 || (D / 512 != 1 && D / 512 != 2 && D / 512 != 4 && D / 512 != 5 && D / 512 != 8))
        return fail(RT_EINVAL, "rt_lm_head_argmax: D must be 512, 1024, 2048, 2560 or 4096");
    DeviceGuard g(ctx->device);
    RT_HIP(launch_lm_head(emb, x, norm_w, eps, V, D, logits, best, token, pos, advance, next_ids, out_tokens, pos_base,
                          out_cap, next_h, ctx->stream));
    return RT_OK;
}

// --- fused decode plans ------------------------------------------------------------

int rt_plan_create_fused(rt_ctx* ctx, int G, const rt_weights* const* w, const rt_src* src, float* const* y,
                         const float* const* residual, rt_plan** out) {
    if (!ctx || !w || !src || !y || !out) return fail(RT_EINVAL, "rt_plan_create_fused: NULL argument");
    *out = nullptr;
    if (G <= 0 || G > (1 << 16)) return fail(RT_EINVAL, "rt_plan_create_fused: G out of range");
    if (!src->x) return fail(RT_EINVAL, "rt_plan_create_fused: source x is NULL");
    if (src->mode != kQuant && src->mode != kRmsNorm && src->mode != kRelu2Mul && src->mode != kRelu2MulNorm &&
        src->mode != kAttnNorm && src->mode != kRmsNormSsq)
        return fail(RT_EINVAL, "rt_plan_create_fused: unknown source mode");
    if (src->mode == kAttnNorm && (src->attn_head_dim <= 0 || src->attn_head_dim % 16 || src->attn_max_len <= 0 ||
                                   !w[0] || w[0]->K % src->attn_head_dim))
        return fail(RT_EINVAL, "rt_plan_create_fused: attention source needs head_dim (multiple of 16) dividing K "
                               "and max_len");
    if ((src->mode != kQuant && !src->aux) ||
        ((src->mode == kRelu2MulNorm || src->mode == kRmsNormSsq) && !src->aux2))
        return fail(RT_EINVAL, "rt_plan_create_fused: the source mode needs aux/aux2");
    const int K = w[0] ? w[0]->K : 0;
    if (src->mode == kRmsNormSsq && (K % 64 || K > 8192))
        return fail(RT_EINVAL, "rt_plan_create_fused: RMSNORM_SSQ needs K % 64 == 0 and K <= 8192");
    for (int g = 0; g < G; ++g) {
        if (!w[g] || !y[g]) return fail(RT_EINVAL, "rt_plan_create_fused: NULL entry in a pointer array");
        if (w[g]->K != K) return fail(RT_EINVAL, "rt_plan_create_fused: all weights must share K (one input)");
        if (w[g]->device != ctx->device) return fail(RT_EINVAL, "rt_plan_create_fused: weights live on another device");
    }
    const int Kp = round_up(K, kChunk);
    if ((size_t)16 * kRowBlock * sizeof(int) + (size_t)Kp + sizeof(double) * 40 > 64 * 1024)
        return fail(RT_EINVAL, "rt_plan_create_fused: K too large for the LDS-resident input row");
    DeviceGuard guard(ctx->device);
    rt_plan* p = new rt_plan();
    p->device = ctx->device;
    p->G = G;
    p->M = 1;
    p->mt = 1;
    p->Mpad = 1;
    p->U = 0;
    p->fused = true;
    p->pro = QuantProb{src->x, nullptr, nullptr, nullptr, nullptr, K, Kp, src->mode, src->aux, src->eps, nullptr,
                       src->aux2, 0, 0};
    if (src->mode == kAttnNorm) {
        p->pro.attn_S = attn_splits(src->attn_max_len);
        p->pro.attn_hd = src->attn_head_dim;
        if ((size_t)(K / src->attn_head_dim) * (p->pro.attn_S + 1) * sizeof(float) > 32 * 1024) {
            rt_plan_free(p);
            return fail(RT_EINVAL, "rt_plan_create_fused: heads x splits too large for the LDS factor table");
        }
    }
    int wg = 0, minC = 1 << 30;
    p->probs.resize(G);
    for (int g = 0; g < G; ++g) {
        p->probs[g] = GemvProb{w[g]->tiles, nullptr, nullptr, nullptr, y[g], w[g]->scale, w[g]->N, w[g]->C, w[g]->N, wg,
                               residual ? residual[g] : nullptr};
        wg += w[g]->Np / kRowBlock;
        if (w[g]->C < minC) minC = w[g]->C;
    }
    p->total_rb = wg;
    p->shape = gemv_shape_fused(wg, minC);
    std::vector<int> rb2p(wg);
    for (int g = 0; g < G; ++g)
        for (int r = 0; r < w[g]->Np / kRowBlock; ++r) rb2p[p->probs[g].wg_begin + r] = g;
    hipError_t e = hipMalloc(&p->dev_probs, sizeof(GemvProb) * G);
    if (e == hipSuccess) e = hipMalloc(&p->dev_rb2p, sizeof(int) * wg);
    if (e == hipSuccess) e = hipMemcpy(p->dev_rb2p, rb2p.data(), sizeof(int) * wg, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p->dev_probs, p->probs.data(), sizeof(GemvProb) * G, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        rt_plan_free(p);
        return hip_fail(e, "rt_plan_create_fused");
    }
    *out = p;
    return RT_OK;
}

int rt_plan_create_gate_up(rt_ctx* ctx, const rt_weights* w_gu, float s_gate, float s_up, const rt_src* src,
                           float* a, double* ssq, float* g_out, float* u_out, rt_plan** out) {
    const char* who = "rt_plan_create_gate_up";
    if (!ctx || !w_gu || !src || !src->x || !a || !ssq || !out)
        return fail(RT_EINVAL, std::string(who) + ": NULL argument");
    *out = nullptr;
    if (src->mode != kQuant && src->mode != kRmsNorm && src->mode != kRmsNormSsq)
        return fail(RT_EINVAL, std::string(who) + ": the source must be QUANT, RMSNORM or RMSNORM_SSQ");
    if ((src->mode != kQuant && !src->aux) || (src->mode == kRmsNormSsq && !src->aux2))
        return fail(RT_EINVAL, std::string(who) + ": the source mode needs aux/aux2");
    if (w_gu->N % kRowBlock) return fail(RT_EINVAL, std::string(who) + ": the interleaved matrix needs N % 64 == 0");
    if (w_gu->device != ctx->device) return fail(RT_EINVAL, std::string(who) + ": weights live on another device");
    const int K = w_gu->K, Kp = round_up(K, kChunk), Nb = w_gu->Np / kRowBlock;
    const GemvShape shape = gemv_shape_fused(Nb, w_gu->C);
    // an E-element prologue (K / 16 <= threads at least), 16-byte aligned rows
    auto a16 = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    if (K % 64 || vec_elements(K, 64 * shape.nw) == 0 || !a16(src->x) || !a16(src->aux) || !a16(src->aux2))
        return fail(RT_EINVAL, std::string(who) + ": needs K % 64 == 0, K / 16 <= the workgroup's threads and "
                                                  "16-byte aligned sources");
    DeviceGuard guard(ctx->device);
    rt_plan* p = new rt_plan();
    p->device = ctx->device;
    p->G = 1;
    p->M = 1;
    p->mt = 1;
    p->Mpad = 1;
    p->U = 0;
    p->fused = true;
    p->pro = QuantProb{src->x, nullptr, nullptr, nullptr, nullptr, K, Kp, src->mode, src->aux, src->eps, nullptr,
                       src->aux2, 0, 0};
    p->probs = {GemvProb{w_gu->tiles, nullptr, nullptr, nullptr, nullptr, w_gu->scale, w_gu->N, w_gu->C, w_gu->N,
                         0, nullptr}};
    p->pair_sg = s_gate;
    p->pair_su = s_up;
    p->total_rb = Nb;
    p->shape = shape;
    p->pair_a = a;
    p->pair_ssq = ssq;
    p->pair_g = g_out;
    p->pair_u = u_out;
    *out = p;
    return RT_OK;
}

// The device state of the attention partials in a qkv launch: the tagged words, the done
// count (epoch 1) and the error count, all zero.
static hipError_t attention_state_reset(rt_plan* plan) {
    hipError_t e = hipMemset(plan->att_mem, 0, plan->att_bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return e;
}

int rt_plan_attach_attention(rt_plan* plan, float* k_cache, float* v_cache, const float* rope, int H, int Hkv,
                             int hd, int Lmax, const int* pos, void* workspace, size_t workspace_bytes) {
    const char* who = "rt_plan_attach_attention";
    if (!plan) return fail(RT_EINVAL, std::string(who) + ": plan is NULL");
    if (!k_cache) {  // detach
        plan->att_on = false;
        return RT_OK;
    }
    if (!v_cache || !rope || !pos || !workspace) return fail(RT_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_heads(H, Hkv, hd, Lmax, who);
    if (rc) return rc;
    if (hd != 128) return fail(RT_EINVAL, std::string(who) + ": head_dim must be 128");
    if (workspace_bytes < rt_attention_decode_workspace(H, hd, Lmax))
        return fail(RT_EINVAL, std::string(who) + ": workspace too small");
    if (!plan->fused || plan->G != 3 || plan->pair_a)
        return fail(RT_EINVAL, std::string(who) + ": needs a fused decode plan of the q, k and v projections "
                                                  "(rt_plan_create_fused, G = 3, RMSNorm or absmax source)");
    const int Gq = H / Hkv;
    if (plan->probs[0].N != H * hd || plan->probs[1].N != Hkv * hd || plan->probs[2].N != Hkv * hd)
        return fail(RT_EINVAL, std::string(who) + ": the plan's outputs must be q [H * hd], k and v [Hkv * hd]");
    // (the poll of an attention workgroup takes one thread per q value of its heads and k, v
    // value of its group: Gq >= 2)
    if (64 * plan->shape.nw != 256 * Gq || Gq < 2)
        return fail(RT_EINVAL, std::string(who) + ": the plan's workgroups must hold one 256-thread attention tile "
                                                  "per query head of a KV group, H / Hkv >= 2 (H / Hkv = 4 for this plan)");
    const QuantProb& P = plan->pro;
    if (P.mode == kAttnNorm || P.K % 64 ||
        vec_elements(P.K, 64 * plan->shape.nw) == 0 || ((uintptr_t)P.x & 15u) || ((uintptr_t)P.aux & 15u))
        return fail(RT_EINVAL, std::string(who) + ": the plan's source must be a 16-byte aligned row with K % 64 == 0");
    DeviceGuard g(plan->device);
    const size_t words = (size_t)(H + 2 * Hkv) * hd;
    const size_t pwords = (size_t)H * attn_splits(Lmax) * (hd + 2);
    // the tagged outputs, the tagged partials (for rt_plan_attention_combine), then done and
    // err
    const size_t bytes = (words + pwords) * sizeof(unsigned long long) + 256;
    // a launch of this plan may still be in flight on the caller's stream: wait for it
    // before the hand-off state is freed or reset
    if (plan->att_mem) RT_HIP(hipDeviceSynchronize());
    if (plan->att_mem && plan->att_bytes != bytes) {
        RT_HIP(hipFree(plan->att_mem));
        plan->att_mem = nullptr;
    }
    if (!plan->att_mem) RT_HIP(hipMalloc(&plan->att_mem, bytes));
    plan->att_bytes = bytes;
    AttnTail& t = plan->att;
    t.tagged = static_cast<unsigned long long*>(plan->att_mem);
    t.ptag = t.tagged + words;
    int* tail = reinterpret_cast<int*>(t.ptag + pwords);
    t.done = reinterpret_cast<unsigned*>(tail);
    t.err = tail + 1;
    t.out = nullptr;  // rt_plan_attention_combine attaches the combine
    t.ssq = nullptr;
    RT_HIP(attention_state_reset(plan));
    t.Kc = k_cache;
    t.Vc = v_cache;
    t.rope = rope;
    t.pos = pos;
    t.work = static_cast<float*>(workspace);
    t.Gq = Gq;
    t.Lmax = Lmax;
    t.S = attn_splits(Lmax);
    // the group's query heads two to a workgroup where they split evenly: the tiles' arithmetic
    // (one CU per workgroup) then spreads over twice the CUs
    t.hpw = Gq % 2 == 0 && Gq >= 4 ? Gq / 2 : Gq;
    t.natt = (unsigned)(Hkv * t.S * (Gq / t.hpw));
    t.wrap = t.natt * (0xFFFFFFFFu / t.natt) - 1u;
    t.qrows = H * hd;
    t.nkv = Hkv * hd;
    t.scale = 1.0f / sqrtf((float)hd);
    plan->att_Hkv = Hkv;
    plan->att_hd = hd;
    plan->att_on = true;
    return RT_OK;
}

int rt_plan_attention_combine(rt_plan* plan, float* out, double* ssq) {
    const char* who = "rt_plan_attention_combine";
    if (!plan) return fail(RT_EINVAL, std::string(who) + ": plan is NULL");
    if (!out != !ssq) return fail(RT_EINVAL, std::string(who) + ": give both out and ssq, or neither");
    if (out) {
        if (!plan->att_on) return fail(RT_EINVAL, std::string(who) + ": attach the attention first "
                                                                     "(rt_plan_attach_attention)");
        if (plan->att.S > kAttnSMax)
            return fail(RT_EINVAL, std::string(who) + ": at most " + std::to_string(kAttnSMax) +
                                       " key blocks (Lmax <= " + std::to_string(64 * kAttnSMax) + ")");
        if (((uintptr_t)out & 15u) || ((uintptr_t)ssq & 7u))
            return fail(RT_EINVAL, std::string(who) + ": out must be 16-byte and ssq 8-byte aligned");
        // the workgroups of a KV group wait for each other's partials: every workgroup of the
        // launch must be resident at once, and a workgroup's chunks of 32 outputs must fit it
        const int NC = plan->att.Gq * plan->att_hd / 32, P = (int)plan->att.natt / plan->att_Hkv;
        if (32 * ((NC + P - 1) / P) > 256 * plan->att.hpw)
            return fail(RT_EINVAL, std::string(who) + ": too few key blocks for the group's outputs");
        DeviceGuard g(plan->device);
        int resident = 0;
        RT_HIP(gemv_attn_capacity(plan->pro.K, plan->pro.Kp, plan->shape.nw, plan->att.Gq, &resident));
        if (plan->total_rb + (int)plan->att.natt > resident)
            return fail(RT_EINVAL, std::string(who) + ": the launch's " +
                                       std::to_string(plan->total_rb + (int)plan->att.natt) +
                                       " workgroups exceed the " + std::to_string(resident) +
                                       " the device holds at once");
    }
    DeviceGuard g(plan->device);
    // a launch of this plan may still be in flight on the caller's stream
    RT_HIP(hipDeviceSynchronize());
    plan->att.out = out;
    plan->att.ssq = ssq;
    return RT_OK;
}

int rt_plan_set_output_ssq(rt_plan* plan, double* ssq) {
    const char* who = "rt_plan_set_output_ssq";
    if (!plan) return fail(RT_EINVAL, std::string(who) + ": plan is NULL");
    if (ssq) {
        if (!plan->fused || plan->G != 1 || plan->M != 1 || plan->pair_a)
            return fail(RT_EINVAL, std::string(who) + ": needs a one-problem fused decode plan "
                                                      "(rt_plan_create_fused, G = 1, not a gate/up pair)");
        if ((uintptr_t)ssq & 7u) return fail(RT_EINVAL, std::string(who) + ": ssq must be 8-byte aligned");
    }
    DeviceGuard g(plan->device);
    // a launch of this plan may still be in flight on the caller's stream
    RT_HIP(hipDeviceSynchronize());
    plan->out_ssq = ssq;
    return RT_OK;
}

int rt_plan_attention_timeouts(rt_plan* plan, int* count) {
    const char* who = "rt_plan_attention_timeouts";
    if (!plan || !count) return fail(RT_EINVAL, std::string(who) + ": NULL argument");
    *count = 0;
    if (!plan->att_mem) return RT_OK;
    DeviceGuard g(plan->device);
    RT_HIP(hipDeviceSynchronize());
    int err = 0;
    RT_HIP(hipMemcpy(&err, plan->att.err, sizeof(int), hipMemcpyDeviceToHost));
    if (err) RT_HIP(attention_state_reset(plan));  // a wait gave up: start again from a clean state
    *count = err;
    return RT_OK;
}

}  // extern "C"
