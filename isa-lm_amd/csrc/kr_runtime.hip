// Device runtime: guard, allocation, copies, the library stream, graphs,
// timers and the sticky error status.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>
#include "kr_internal.h"

static int g_ready = 0;
static hipStream_t g_stream = nullptr;
static char g_arch[64] = "";
static int g_cus = 0;
static ml_status g_status = ML_OK;
static char g_msg[512] = "";

hipStream_t kr_stream(void) { return g_stream; }

void kr_fail(ml_status st, const char *what, hipError_t e) {
    if (g_status != ML_OK) return;
    g_status = st;
    snprintf(g_msg, sizeof g_msg, "%s: %s", what, e == hipSuccess ? "invalid argument" : hipGetErrorString(e));
}

void kr_check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) kr_fail(ML_E_SHAPE, what, e);
}

extern "C" ml_status krh_init(void) {
    if (g_ready) return ML_OK;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        snprintf(g_msg, sizeof g_msg, "no HIP device");
        return ML_E_ISA;
    }
    hipDeviceProp_t p;
    if (hipSetDevice(0) != hipSuccess || hipGetDeviceProperties(&p, 0) != hipSuccess) {
        snprintf(g_msg, sizeof g_msg, "cannot open HIP device 0");
        return ML_E_ISA;
    }
    snprintf(g_arch, sizeof g_arch, "%s", p.gcnArchName);
    g_cus = p.multiProcessorCount;
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        snprintf(g_msg, sizeof g_msg, "device 0 is %s, this build needs gfx950", p.gcnArchName);
        return ML_E_ISA;
    }
    if (kr_attn_setup(0) != ML_OK) {
        snprintf(g_msg, sizeof g_msg, "cannot take the address of the attention scratch array");
        return ML_E_ISA;
    }
    if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) {
        snprintf(g_msg, sizeof g_msg, "cannot create a stream");
        return ML_E_ISA;
    }
    g_ready = 1;
    return ML_OK;
}

extern "C" const char *krh_device_arch(void) { return g_arch; }
extern "C" int krh_device_cus(void) { return g_cus; }
extern "C" ml_status krh_status(void) { return g_status; }
extern "C" const char *krh_last_error(void) { return g_msg; }
extern "C" void krh_clear_error(void) { g_status = ML_OK; g_msg[0] = 0; }

extern "C" void *krh_alloc(size_t bytes) {
    void *p = nullptr;
    if (!g_ready || hipMalloc(&p, bytes ? bytes : 256) != hipSuccess) return nullptr;
    return p;
}
extern "C" void krh_free(void *p) { if (p) (void)hipFree(p); }
extern "C" void *krh_host_alloc(size_t bytes) {
    void *p = nullptr;
    if (!g_ready || hipHostMalloc(&p, bytes ? bytes : 64, hipHostMallocDefault) != hipSuccess) return nullptr;
    return p;
}
extern "C" void krh_host_free(void *p) { if (p) (void)hipHostFree(p); }

extern "C" ml_status krh_copy_h2d(void *dst, const void *src, size_t bytes) {
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream);
    if (e != hipSuccess) { kr_fail(ML_E_IO, "copy to device", e); return ML_E_IO; }
    return krh_sync();
}
extern "C" ml_status krh_copy_d2h(void *dst, const void *src, size_t bytes) {
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream);
    if (e != hipSuccess) { kr_fail(ML_E_IO, "copy to host", e); return ML_E_IO; }
    return krh_sync();
}
extern "C" void krh_copy_d2d_async(void *dst, const void *src, size_t bytes) {
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream);
    if (e != hipSuccess) kr_fail(ML_E_IO, "device copy", e);
}
extern "C" ml_status krh_sync(void) {
    const hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) kr_fail(ML_E_IO, "device fault", e);
    return g_status;
}

struct krh_graph { hipGraph_t g; hipGraphExec_t x; };

extern "C" ml_status krh_graph_begin(void) {
    const hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) { kr_fail(ML_E_IO, "begin capture", e); return ML_E_IO; }
    return ML_OK;
}
extern "C" ml_status krh_graph_end(krh_graph **out) {
    krh_graph *g = new krh_graph();
    hipError_t e = hipStreamEndCapture(g_stream, &g->g);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->x, g->g, nullptr, nullptr, 0);
    if (e != hipSuccess) { kr_fail(ML_E_IO, "graph capture", e); delete g; *out = nullptr; return ML_E_IO; }
    *out = g;
    return g_status;
}
extern "C" ml_status krh_graph_launch(const krh_graph *g) {
    const hipError_t e = hipGraphLaunch(g->x, g_stream);
    if (e != hipSuccess) { kr_fail(ML_E_IO, "graph launch", e); return ML_E_IO; }
    return ML_OK;
}
extern "C" void krh_graph_free(krh_graph *g) {
    if (!g) return;
    (void)hipGraphExecDestroy(g->x);
    (void)hipGraphDestroy(g->g);
    delete g;
}

struct krh_timer { hipEvent_t e[2]; };
extern "C" krh_timer *krh_timer_new(void) {
    krh_timer *t = new krh_timer();
    (void)hipEventCreate(&t->e[0]);
    (void)hipEventCreate(&t->e[1]);
    return t;
}
extern "C" void krh_timer_mark(krh_timer *t, int which) { (void)hipEventRecord(t->e[which ? 1 : 0], g_stream); }
extern "C" float krh_timer_ms(krh_timer *t) {
    float ms = 0.0f;
    (void)hipEventSynchronize(t->e[1]);
    (void)hipEventElapsedTime(&ms, t->e[0], t->e[1]);
    return ms;
}
extern "C" void krh_timer_free(krh_timer *t) {
    if (!t) return;
    (void)hipEventDestroy(t->e[0]);
    (void)hipEventDestroy(t->e[1]);
    delete t;
}
