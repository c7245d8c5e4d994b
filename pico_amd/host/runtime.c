/*
 * pico_amd/host/runtime.c -- device bring-up, the library's stream, error
 * reporting and device memory helpers for libpico_amd.so.
 *
 * pico's pico_init (src/global.c:29-69) selects a SIMD level, a GPU enum and
 * starts its thread pool; here it selects the HIP device ($PICO_DEVICE, else
 * 0) and creates one non-blocking stream at default priority that every
 * launch of this library uses.
 */
#include <hip/hip_runtime_api.h>
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

#include "pk_host.h"

uint32_t x_state = 123456789u; /* src/global.c:13 */

static int g_ready = 0;
static int g_device = 0;
static hipStream_t g_own_stream = NULL;
static hipStream_t g_user_stream = NULL;
static int g_user_stream_set = 0;
static char g_err[512] = "";

/* graph capture: while set, every launch is recorded on the library's stream,
 * and anything that would allocate, free, copy synchronously or wait on the
 * device fails the capture instead */
static int g_capturing = 0;
static int g_capture_failed = 0;

static void* g_ws = NULL;
static size_t g_ws_bytes = 0;

/* the side stream (weight gradients), its fork/join events and scratch */
static hipStream_t g_side = NULL;
static hipEvent_t g_fork_ev = NULL, g_join_ev = NULL;
static uint64_t g_side_seq = 0, g_side_joined = 0;
static int g_side_broken = 0;
static void* g_side_ws = NULL;
static size_t g_side_ws_bytes = 0;

static uint64_t g_err_count = 0;

void pkh_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    g_err_count++;
}

uint64_t pkh_error_count(void) { return g_err_count; }

/* refuses a call that cannot be recorded in a graph; returns nonzero then */
static int capture_refuses(const char* what) {
    if(!g_capturing) return 0;
    g_capture_failed = 1;
    pkh_set_error("%s during graph capture: run the step once before capturing, pass "
                  "token ids as device pointers, and read results after pico_graph_launch",
                  what);
    PKH_ERR("%s\n", g_err);
    return 1;
}

int pkh_capturing(void) { return g_capturing; }

int pkh_init(void) {
    if(g_ready) return 0;
    const char* env = getenv("PICO_DEVICE");
    g_device = env ? atoi(env) : 0;
    hipError_t e = hipSetDevice(g_device);
    if(e == hipSuccess) e = hipStreamCreateWithFlags(&g_own_stream, hipStreamNonBlocking);
    if(e != hipSuccess) {
        pkh_set_error("pico_init: HIP device %d unavailable: %s", g_device, hipGetErrorString(e));
        PKH_ERR("%s\n", g_err);
        return (int)e;
    }
    g_ready = 1;
    return 0;
}

void pico_init(void) { (void)pkh_init(); }

void pico_shutdown(void) {
    if(!g_ready) return;
    pkh_side_join();
    hipStreamSynchronize(g_own_stream);
    pkh_mx8_release();
    if(g_ws) pkh_device_free(g_ws);
    g_ws = NULL;
    g_ws_bytes = 0;
    if(g_side) {
        if(g_side_ws) pkh_device_free(g_side_ws);
        g_side_ws = NULL;
        g_side_ws_bytes = 0;
        hipEventDestroy(g_fork_ev);
        hipEventDestroy(g_join_ev);
        hipStreamDestroy(g_side);
        g_side = NULL;
    }
    hipStreamDestroy(g_own_stream);
    g_own_stream = NULL;
    g_ready = 0;
}

pk_stream_t pkh_stream(void) {
    return (pk_stream_t)(g_user_stream_set ? g_user_stream : g_own_stream);
}

void* pico_gpu_stream(void) {
    pkh_init();
    return (void*)pkh_stream();
}

void pico_gpu_set_stream(void* stream) {
    g_user_stream = (hipStream_t)stream;
    g_user_stream_set = stream != NULL;
}

int pkh_status(const char* op, int status) {
    if(status == 0) return 0;
    if(g_capturing) g_capture_failed = 1;
    const char* msg = pk_last_error();
    if(status != PK_EINVAL || !msg || !*msg) msg = hipGetErrorString((hipError_t)status);
    pkh_set_error("%s: %s (status %d)", op, msg, status);
    PKH_ERR("%s\n", g_err);
    return status;
}

/* Graph capture and the side stream.  A replay runs the captured graph's
 * branches on several streams, and a node's stream continues with its first
 * captured child (ROCm's executor walks the graph depth first along first
 * children).  At an eager fork the side-stream work is issued first, so
 * captured the same way the weight-gradient chain would take the launch
 * stream and the critical path's kernels would queue behind it (measured:
 * RMSNorm's backward waiting for weight-gradient products, config 4's replay
 * 8 % slower than its eager step).  So under capture a fork is taken in two
 * steps, with the main stream's next kernel captured in between:
 * pkh_side_prepare() records the fork point on the main stream, the caller
 * issues its main-stream kernel, then pkh_side_fork() makes the side stream
 * wait for the prepared point (not for that kernel).  Side work that has no
 * main-stream kernel of its own to follow (RMSNorm's gain reduction, a
 * bias gradient) is deferred under capture (pkh_side_defer) and issued at the
 * next fork or join. */
static int g_prepared = 0;

struct SideJob {
    pkh_side_job_fn fn;
    unsigned char args[PKH_SIDE_JOB_ARGS];
};
static struct SideJob g_jobs[64];
static int g_njobs = 0;

static int side_create(void) {
    if(g_side) return 0;
    /* default priority, like the main stream */
    hipError_t e = hipStreamCreateWithFlags(&g_side, hipStreamNonBlocking);
    if(e == hipSuccess) e = hipEventCreateWithFlags(&g_fork_ev, hipEventDisableTiming);
    if(e == hipSuccess) e = hipEventCreateWithFlags(&g_join_ev, hipEventDisableTiming);
    if(e != hipSuccess) {
        (void)hipGetLastError();
        g_side_broken = 1;
        return -1;
    }
    return 0;
}

int pkh_side_prepare(void) {
    if(!g_capturing || pkh_init() || g_side_broken || side_create()) return 0;
    if(hipEventRecord(g_fork_ev, (hipStream_t)pkh_stream()) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    g_prepared = 1;
    return 1;
}

pk_stream_t pkh_side_fork(void) {
    if(pkh_init() || g_side_broken || side_create()) return NULL;
    hipError_t e = hipSuccess;
    if(!g_prepared) e = hipEventRecord(g_fork_ev, (hipStream_t)pkh_stream());
    g_prepared = 0;
    if(e == hipSuccess) e = hipStreamWaitEvent(g_side, g_fork_ev, 0);
    if(e != hipSuccess) {
        pkh_status("side stream fork", (int)e);
        return NULL;
    }
    ++g_side_seq;
    /* side work deferred under capture goes first on the side stream */
    for(int i = 0; i < g_njobs; i++) g_jobs[i].fn(g_jobs[i].args, (pk_stream_t)g_side);
    g_njobs = 0;
    return (pk_stream_t)g_side;
}

int pkh_side_defer(pkh_side_job_fn fn, const void* args, size_t n) {
    if(!g_capturing || n > PKH_SIDE_JOB_ARGS || pkh_init() || g_side_broken) return 0;
    if(g_njobs == (int)(sizeof(g_jobs) / sizeof(g_jobs[0]))) {
        if(!pkh_side_fork()) return 0; /* issues the queued jobs */
    }
    g_jobs[g_njobs].fn = fn;
    memcpy(g_jobs[g_njobs].args, args, n);
    g_njobs++;
    return 1;
}

uint64_t pkh_side_seq(void) { return g_side_seq; }
uint64_t pkh_side_joined(void) { return g_side_joined; }

void pkh_side_join(void) {
    if(g_njobs) pkh_side_fork(); /* issue deferred side work first */
    if(g_side_joined == g_side_seq) return;
    hipError_t e = hipEventRecord(g_join_ev, g_side);
    if(e == hipSuccess) e = hipStreamWaitEvent((hipStream_t)pkh_stream(), g_join_ev, 0);
    if(e != hipSuccess) {
        /* cannot order the streams: wait for the side stream from the host */
        pkh_status("side stream join", (int)e);
        hipStreamSynchronize(g_side);
    }
    g_side_joined = g_side_seq;
}

static void* device_alloc(size_t bytes, int quiet);
static int g_fail_opt_ws = 0; /* pico_gpu_fail_next_workspaces */

/* a scratch buffer of at least `bytes` in *buf, grown (after the stream that
 * may still read the old one is done) when smaller.  `optional`: the caller
 * has a fallback without it, so a failed allocation records no error (it
 * would otherwise stop pico_backward) and returns NULL. */
static void* grow_workspace(void** buf, size_t* have, hipStream_t st, size_t bytes, int optional,
                            const char* what) {
    if(optional && g_fail_opt_ws > 0) {
        g_fail_opt_ws--;
        return NULL;
    }
    if(bytes <= *have) return *buf;
    if(capture_refuses(what)) return NULL;
    if(*buf) {
        hipStreamSynchronize(st);
        pkh_device_free(*buf);
        *buf = NULL;
        *have = 0;
    }
    *buf = device_alloc(bytes, optional);
    if(*buf) *have = bytes;
    return *buf;
}

void* pkh_side_workspace(size_t bytes) {
    return grow_workspace(&g_side_ws, &g_side_ws_bytes, g_side, bytes, 0,
                          "growing the side-stream workspace");
}

void* pkh_side_workspace_opt(size_t bytes) {
    return grow_workspace(&g_side_ws, &g_side_ws_bytes, g_side, bytes, 1,
                          "growing the side-stream workspace");
}

void pico_gpu_fail_next_workspaces(int n) { g_fail_opt_ws = n > 0 ? n : 0; }

int pkh_sync(void) {
    if(pkh_init()) return -1;
    if(capture_refuses("waiting on the device")) return -1;
    pkh_side_join();
    hipError_t e = hipStreamSynchronize((hipStream_t)pkh_stream());
    if(e != hipSuccess) return pkh_status("pico_gpu_synchronize", (int)e);
    return 0;
}

int pico_gpu_synchronize(void) { return pkh_sync(); }
const char* pico_gpu_last_error(void) { return g_err; }
void pico_gpu_clear_error(void) { g_err[0] = 0; }

static size_t g_dev_bytes = 0, g_dev_peak = 0;

/* quiet: a failure is the caller's to handle; it records no error and
 * clears HIP's sticky status, so the next launch check does not see it */
static void* device_alloc(size_t bytes, int quiet) {
    if(pkh_init()) return NULL;
    if(capture_refuses("device allocation")) return NULL;
    void* p = NULL;
    if(!bytes) bytes = 256;
    hipError_t e = hipMalloc(&p, bytes);
    if(e != hipSuccess) {
        (void)hipGetLastError();
        if(quiet) return NULL;
        pkh_set_error("device allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
        PKH_ERR("%s\n", g_err);
        return NULL;
    }
    g_dev_bytes += bytes;
    if(g_dev_bytes > g_dev_peak) g_dev_peak = g_dev_bytes;
    return p;
}

void* pkh_device_alloc(size_t bytes) { return device_alloc(bytes, 0); }

void pkh_device_free(void* p) {
    if(!p) return;
    if(capture_refuses("freeing device memory")) return;
    size_t sz = 0;
    if(hipMemPtrGetInfo(p, &sz) == hipSuccess) g_dev_bytes -= sz < g_dev_bytes ? sz : g_dev_bytes;
    hipFree(p);
}

void pico_gpu_memory(size_t* in_use, size_t* peak) {
    if(in_use) *in_use = g_dev_bytes;
    if(peak) *peak = g_dev_peak;
}

void* pkh_workspace(size_t bytes) {
    return grow_workspace(&g_ws, &g_ws_bytes, (hipStream_t)pkh_stream(), bytes, 0,
                          "growing the GEMM workspace");
}

void* pkh_workspace_opt(size_t bytes) {
    return grow_workspace(&g_ws, &g_ws_bytes, (hipStream_t)pkh_stream(), bytes, 1,
                          "growing the GEMM workspace");
}

int pkh_is_device_ptr(const void* p) {
    if(!p || pkh_init()) return 0;
    hipPointerAttribute_t attr;
    memset(&attr, 0, sizeof(attr));
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if(e != hipSuccess) {
        (void)hipGetLastError(); /* plain host memory: clear the sticky status */
        return 0;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

int pkh_copy_h2d(void* dst, const void* src, size_t bytes) {
    if(pkh_init()) return -1;
    if(capture_refuses("a host-to-device copy")) return -1;
    if(bytes == 0) return 0;
    pkh_params_changed(); /* the copy may write a parameter */
    pkh_side_join();
    hipStream_t st = (hipStream_t)pkh_stream();
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
    if(e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? 0 : pkh_status("host-to-device copy", (int)e);
}

int pkh_copy_d2h(void* dst, const void* src, size_t bytes) {
    if(pkh_init()) return -1;
    if(capture_refuses("a device-to-host copy")) return -1;
    if(bytes == 0) return 0;
    pkh_side_join();
    hipStream_t st = (hipStream_t)pkh_stream();
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st);
    if(e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? 0 : pkh_status("device-to-host copy", (int)e);
}

int pkh_copy_d2d_async(void* dst, const void* src, size_t bytes) {
    if(bytes == 0) return 0;
    pkh_params_changed(); /* the copy may write a parameter */
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                                  (hipStream_t)pkh_stream());
    return e == hipSuccess ? 0 : pkh_status("device-to-device copy", (int)e);
}

/* ------------------------------------------------------------ device graphs */
struct PicoGraph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

int pico_graph_begin(void) {
    if(pkh_init()) return -1;
    if(g_capturing) {
        pkh_set_error("pico_graph_begin: a capture is already in progress");
        PKH_ERR("%s\n", g_err);
        return PK_EINVAL;
    }
    /* relaxed: the library itself refuses every call that would break the
     * graph (see capture_refuses) */
    hipError_t e = hipStreamBeginCapture((hipStream_t)pkh_stream(), hipStreamCaptureModeRelaxed);
    if(e != hipSuccess) return pkh_status("pico_graph_begin", (int)e);
    g_capturing = 1;
    g_capture_failed = 0;
    /* kept fp8 casts are redone inside the graph, so every replay recasts */
    pkh_params_changed();
    return 0;
}

struct PicoGraph* pico_graph_end(void) {
    if(!g_capturing) {
        pkh_set_error("pico_graph_end: no capture in progress");
        PKH_ERR("%s\n", g_err);
        return NULL;
    }
    pkh_side_join(); /* the side stream's work joins the captured graph */
    hipGraph_t graph = NULL;
    hipError_t e = hipStreamEndCapture((hipStream_t)pkh_stream(), &graph);
    g_capturing = 0;
    pkh_params_changed(); /* the casts captured were never run */
    if(e != hipSuccess || g_capture_failed) {
        if(graph) hipGraphDestroy(graph);
        if(e != hipSuccess) pkh_status("pico_graph_end", (int)e);
        return NULL;
    }
    struct PicoGraph* g = (struct PicoGraph*)calloc(1, sizeof(*g));
    if(!g) {
        hipGraphDestroy(graph);
        pkh_set_error("pico_graph_end: out of host memory");
        return NULL;
    }
    g->graph = graph;
    e = hipGraphInstantiate(&g->exec, graph, NULL, NULL, 0);
    if(e != hipSuccess) {
        hipGraphDestroy(graph);
        free(g);
        pkh_status("pico_graph_end (instantiate)", (int)e);
        return NULL;
    }
    return g;
}

int pico_graph_launch(struct PicoGraph* g) {
    if(!g) {
        pkh_set_error("pico_graph_launch: NULL graph");
        return PK_EINVAL;
    }
    if(g_capturing) {
        pkh_set_error("pico_graph_launch: cannot launch a graph while capturing");
        return PK_EINVAL;
    }
    hipError_t e = hipGraphLaunch(g->exec, (hipStream_t)pkh_stream());
    pkh_params_changed(); /* a replayed step may update parameters */
    return e == hipSuccess ? 0 : pkh_status("pico_graph_launch", (int)e);
}

void pico_graph_free(struct PicoGraph* g) {
    if(!g) return;
    hipStreamSynchronize((hipStream_t)pkh_stream());
    hipGraphExecDestroy(g->exec);
    hipGraphDestroy(g->graph);
    free(g);
}
