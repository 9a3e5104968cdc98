// Context, stream, memory and error handling of libvx27_hip.
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <unordered_map>

#include "vx_common.h"
#include "vx_gqa.h"

static thread_local char g_err[512] = "";

void vx_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

extern "C" const char *vx27_hip_last_error(void) { return g_err; }

extern "C" const char *vx27_hip_version(void) { return "vx27_hip 0.1 gfx950"; }

extern "C" int vx27_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int vx_ctx_enter(vx27_hip_ctx *ctx) {
    VX_REQUIRE(ctx != nullptr, "null context");
    VX_HIP(hipSetDevice(ctx->device));
    return 0;
}

extern "C" int vx27_hip_open(vx27_hip_ctx **out, int device, char *err, size_t errlen) {
    auto fail = [&](void) {
        if (err && errlen) snprintf(err, errlen, "%s", g_err);
        return -1;
    };
    if (!out) {
        vx_set_error("vx27_hip_open: null output pointer");
        return fail();
    }
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        vx_set_error("vx27_hip_open: no HIP device (%s)", hipGetErrorString(e));
        return fail();
    }
    if (device < 0 || device >= n) {
        vx_set_error("vx27_hip_open: device %d out of range (have %d)", device, n);
        return fail();
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        vx_set_error("vx27_hip_open: cannot query device %d", device);
        return fail();
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        vx_set_error("vx27_hip_open: device %d is %s; this library is built for gfx950", device,
                     prop.gcnArchName);
        return fail();
    }
    vx27_hip_ctx *c = new vx27_hip_ctx();
    c->device = device;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) {
        vx_set_error("vx27_hip_open: stream creation failed on device %d", device);
        delete c;
        return fail();
    }
    if (hipMalloc((void **)&c->err_flag, 256) != hipSuccess || hipMemset(c->err_flag, 0, 256) != hipSuccess ||
        hipHostMalloc((void **)&c->err_host, 256, hipHostMallocDefault) != hipSuccess) {
        vx_set_error("vx27_hip_open: cannot allocate the error flag on device %d", device);
        if (c->err_flag) (void)hipFree(c->err_flag);
        if (c->err_host) (void)hipHostFree(c->err_host);
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return fail();
    }
    *c->err_host = 0;
    if (vx_noalloc_init(device) != 0) {
        (void)hipHostFree(c->err_host);
        (void)hipFree(c->err_flag);
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return fail();
    }
    c->stream = c->own_stream;
    c->n_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    *out = c;
    return 0;
}

static void prof_clear(vx27_hip_ctx *ctx) {
    for (int i = 0; i < ctx->prof_n; i++) {
        (void)hipEventDestroy(ctx->prof[i].e0);
        (void)hipEventDestroy(ctx->prof[i].e1);
    }
    ctx->prof_n = 0;
}

void vx_prof_begin(vx27_hip_ctx *ctx) {
    if (!ctx->prof_on) return;
    if (ctx->prof_n == ctx->prof_cap) {
        int cap = ctx->prof_cap ? 2 * ctx->prof_cap : 256;
        vx_prof_rec *p = (vx_prof_rec *)realloc(ctx->prof, sizeof(vx_prof_rec) * (size_t)cap);
        if (!p) return;
        ctx->prof = p;
        ctx->prof_cap = cap;
    }
    vx_prof_rec *r = &ctx->prof[ctx->prof_n];
    r->name = nullptr;
    if (hipEventCreate(&r->e0) != hipSuccess) return;
    if (hipEventCreate(&r->e1) != hipSuccess) {
        (void)hipEventDestroy(r->e0);
        return;
    }
    (void)hipEventRecord(r->e0, ctx->stream);
    ctx->prof_n++;
}

void vx_prof_end(vx27_hip_ctx *ctx, const char *name) {
    if (!ctx->prof_on || ctx->prof_n == 0) return;
    vx_prof_rec *r = &ctx->prof[ctx->prof_n - 1];
    if (r->name) return;   // begin failed
    r->name = name;
    (void)hipEventRecord(r->e1, ctx->stream);
}

extern "C" int vx27_hip_prof_enable(vx27_hip_ctx *ctx, int on) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_HIP(hipStreamSynchronize(ctx->stream));
    prof_clear(ctx);
    ctx->prof_on = on ? 1 : 0;
    return 0;
}

extern "C" int vx27_hip_prof_read(vx27_hip_ctx *ctx, const char *name, int *count, double *total_ms) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(name && count && total_ms, "vx27_hip_prof_read: null argument");
    VX_HIP(hipStreamSynchronize(ctx->stream));
    int n = 0;
    double tot = 0.0;
    for (int i = 0; i < ctx->prof_n; i++) {
        const vx_prof_rec *r = &ctx->prof[i];
        // a template's instances (kernel<1>, kernel<4>, ...) count under its name
        const size_t ln = strlen(name);
        if (!r->name || strncmp(r->name, name, ln) != 0 || (r->name[ln] != '\0' && r->name[ln] != '<'))
            continue;
        float ms = 0.0f;
        VX_HIP(hipEventElapsedTime(&ms, r->e0, r->e1));
        tot += ms;
        n++;
    }
    *count = n;
    *total_ms = tot;
    return 0;
}

static void graphs_forget(vx27_hip_ctx *ctx);

extern "C" void vx27_hip_close(vx27_hip_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    graphs_forget(ctx);
    prof_clear(ctx);
    free(ctx->prof);
    vx_gqp_sched_free(ctx);
    for (void *p : ctx->retired) (void)hipFree(p);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->stage) (void)hipFree(ctx->stage);
    if (ctx->err_flag) (void)hipFree(ctx->err_flag);
    if (ctx->err_host) (void)hipHostFree(ctx->err_host);
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

extern "C" int vx27_hip_sync(vx27_hip_ctx *ctx) {
    if (vx_ctx_enter(ctx)) return -1;
    // the flag's copy rides on the stream, so one wait covers both
    VX_HIP(hipMemcpyAsync(ctx->err_host, ctx->err_flag, sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
    VX_HIP(hipStreamSynchronize(ctx->stream));
    const int flag = *(volatile int *)ctx->err_host;
    if (flag) {
        *ctx->err_host = 0;
        VX_HIP(hipMemcpyAsync(ctx->err_flag, ctx->err_host, sizeof(int), hipMemcpyHostToDevice, ctx->stream));
        VX_HIP(hipStreamSynchronize(ctx->stream));
        VX_REQUIRE(false, "vx27_hip_sync: a call since the last sync had an index outside its range (a decode "
                          "position outside its KV cache, or a commit index past its checkpoints); that call's "
                          "outputs are undefined");
    }
    return 0;
}

extern "C" int vx27_hip_set_stream(vx27_hip_ctx *ctx, void *s) {
    VX_REQUIRE(ctx != nullptr, "null context");
    ctx->stream = s ? (hipStream_t)s : ctx->own_stream;
    return 0;
}

extern "C" void *vx27_hip_get_stream(vx27_hip_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

bool vx_ctx_capturing(vx27_hip_ctx *ctx) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cs) != hipSuccess) return true;
    return cs != hipStreamCaptureStatusNone;
}

static std::mutex g_graph_mu;   // guards live_graphs and the owner map below

void vx_ctx_release(vx27_hip_ctx *ctx, void *dptr) {
    if (!dptr) return;
    std::lock_guard<std::mutex> lk(g_graph_mu);
    if (ctx->live_graphs > 0)
        ctx->retired.push_back(dptr);
    else
        (void)hipFree(dptr);
}

int vx_ctx_scratch(vx27_hip_ctx *ctx, size_t bytes, void **out) {
    if (bytes > ctx->scratch_bytes) {
        VX_REQUIRE(!vx_ctx_capturing(ctx),
                   "scratch of %zu bytes needed inside a graph capture (have %zu): run the same call once "
                   "before capturing",
                   bytes, ctx->scratch_bytes);
        VX_HIP(hipStreamSynchronize(ctx->stream));
        vx_ctx_release(ctx, ctx->scratch);
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
        size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
        VX_HIP(hipMalloc(&ctx->scratch, want));
        ctx->scratch_bytes = want;
    }
    *out = ctx->scratch;
    return 0;
}

// ------------------------------------------------------------- HIP graphs
// Which context captured each live executable graph (graph_destroy has no
// context argument).
static std::unordered_map<void *, vx27_hip_ctx *> g_graph_owner;

static void graphs_forget(vx27_hip_ctx *ctx) {
    std::lock_guard<std::mutex> lk(g_graph_mu);
    for (auto &kv : g_graph_owner)
        if (kv.second == ctx) kv.second = nullptr;
}

extern "C" int vx27_hip_graph_begin(vx27_hip_ctx *ctx) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(!ctx->prof_on, "vx27_hip_graph_begin: disable the profiler before capturing");
    VX_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return 0;
}

extern "C" int vx27_hip_graph_end(vx27_hip_ctx *ctx, void **graph_exec) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(graph_exec != nullptr, "vx27_hip_graph_end: null output");
    hipGraph_t g = nullptr;
    VX_HIP(hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t e = nullptr;
    const hipError_t rc = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    VX_HIP(rc);
    {
        std::lock_guard<std::mutex> lk(g_graph_mu);
        g_graph_owner[(void *)e] = ctx;
        ctx->live_graphs++;
    }
    *graph_exec = (void *)e;
    return 0;
}

extern "C" int vx27_hip_graph_launch(vx27_hip_ctx *ctx, void *graph_exec) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(graph_exec != nullptr, "vx27_hip_graph_launch: null graph");
    VX_HIP(hipGraphLaunch((hipGraphExec_t)graph_exec, ctx->stream));
    return 0;
}

extern "C" int vx27_hip_graph_destroy(void *graph_exec) {
    if (!graph_exec) return 0;
    vx27_hip_ctx *owner = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_graph_mu);
        auto it = g_graph_owner.find(graph_exec);
        if (it != g_graph_owner.end()) {
            owner = it->second;
            g_graph_owner.erase(it);
        }
    }
    if (owner) {
        VX_HIP(hipSetDevice(owner->device));
        // a replay of this graph may still be running on the stream
        VX_HIP(hipStreamSynchronize(owner->stream));
    }
    VX_HIP(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
    if (owner) {
        std::vector<void *> drop;
        {
            std::lock_guard<std::mutex> lk(g_graph_mu);
            if (--owner->live_graphs == 0) drop.swap(owner->retired);
        }
        for (void *p : drop) VX_HIP(hipFree(p));
    }
    return 0;
}

int vx_ctx_stage(vx27_hip_ctx *ctx, size_t bytes, void **out) {
    if (bytes > ctx->stage_bytes) {
        VX_HIP(hipStreamSynchronize(ctx->stream));
        if (ctx->stage) VX_HIP(hipFree(ctx->stage));
        ctx->stage = nullptr;
        ctx->stage_bytes = 0;
        size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
        VX_HIP(hipMalloc(&ctx->stage, want));
        ctx->stage_bytes = want;
    }
    *out = ctx->stage;
    return 0;
}

// ------------------------------------------------------------------ memory
extern "C" int vx27_hip_alloc(vx27_hip_ctx *ctx, void **dptr, size_t bytes) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(dptr != nullptr, "vx27_hip_alloc: null output pointer");
    *dptr = nullptr;
    VX_HIP(hipMalloc(dptr, bytes ? bytes : 1));
    return 0;
}
extern "C" int vx27_hip_free(vx27_hip_ctx *ctx, void *dptr) {
    if (vx_ctx_enter(ctx)) return -1;
    if (dptr) {
        VX_HIP(hipStreamSynchronize(ctx->stream));
        VX_HIP(hipFree(dptr));
    }
    return 0;
}
extern "C" int vx27_hip_h2d(vx27_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    VX_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}
extern "C" int vx27_hip_d2h(vx27_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    VX_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}
extern "C" int vx27_hip_d2d(vx27_hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return 0;
}
// A byte fill as a kernel, not hipMemsetAsync, so that a caller may capture
// it into a graph: the bytes before the first 16-byte boundary and after the
// last one are stored singly, the rest as 16-byte vector stores.
__global__ __launch_bounds__(256) void vx_fill_kernel(unsigned char *dst, size_t head, size_t n16, size_t tail,
                                                      uint32_t word) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
    const uint4 w4 = make_uint4(word, word, word, word);
    uint4 *body = (uint4 *)(dst + head);
    for (size_t j = i; j < n16; j += stride) body[j] = w4;
    if (i < head) dst[i] = (unsigned char)word;
    if (i < tail) dst[head + n16 * 16 + i] = (unsigned char)word;
}

extern "C" int vx27_hip_memset(vx27_hip_ctx *ctx, void *dst, int byte, size_t bytes) {
    if (vx_ctx_enter(ctx)) return -1;
    if (bytes == 0) return 0;
    VX_REQUIRE(dst != nullptr, "vx27_hip_memset: null pointer");
    const uintptr_t a = (uintptr_t)dst;
    size_t head = (16 - (a & 15)) & 15;
    if (head > bytes) head = bytes;
    const size_t n16 = (bytes - head) / 16, tail = bytes - head - n16 * 16;
    const uint32_t word = 0x01010101u * (uint32_t)(unsigned char)byte;
    const size_t want = (n16 + 255) / 256;
    const unsigned grid = (unsigned)(want < 1 ? 1 : want > 4096 ? 4096 : want);
    VX_LAUNCH(ctx, vx_fill_kernel, dim3(grid), dim3(256), (unsigned char *)dst, head, n16, tail, word);
    return 0;
}

extern "C" int vx27_hip_mem_info(vx27_hip_ctx *ctx, size_t *scratch_bytes, int *retired_buffers,
                                 int *cached_schedules, int *live_graphs) {
    VX_REQUIRE(ctx != nullptr, "null context");
    std::lock_guard<std::mutex> lk(g_graph_mu);
    if (scratch_bytes) *scratch_bytes = ctx->scratch_bytes;
    if (retired_buffers) *retired_buffers = (int)ctx->retired.size();
    if (cached_schedules) *cached_schedules = (int)ctx->gqp_scheds.size();
    if (live_graphs) *live_graphs = ctx->live_graphs;
    return 0;
}

// ------------------------------------------------ default (drop-in) context
static vx27_hip_ctx *g_default = nullptr;
static int g_errmode = VX27_HIP_ERR_ABORT;

extern "C" void vx27_hip_set_error_mode(int mode) { g_errmode = mode; }
extern "C" int vx27_hip_get_error_mode(void) { return g_errmode; }

static std::atomic<int> g_route_on{0};

extern "C" int vx27_hip_enable(void) {
    if (!vx27_hip_default_ctx()) return -1;
    g_route_on.store(1);
    return 0;
}
extern "C" void vx27_hip_disable(void) { g_route_on.store(0); }
extern "C" int vx27_hip_enabled(void) { return g_route_on.load(); }

// Opened once, by the first caller, whichever thread that is.
static std::once_flag g_default_once;

extern "C" vx27_hip_ctx *vx27_hip_default_ctx(void) {
    std::call_once(g_default_once, [] {
        const char *env = getenv("VX27_HIP_DEVICE");
        int dev = env ? atoi(env) : 0;
        char err[256];
        if (vx27_hip_open(&g_default, dev, err, sizeof err) != 0) g_default = nullptr;
    });
    if (!g_default) vx_set_error("vx27_hip_default_ctx: no context could be opened on the default device");
    return g_default;
}
