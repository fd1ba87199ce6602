/*
 * runtime.hip - device, memory, stream, events and graph capture of the HIP
 * layer (role of iris_metal.m's runtime: init, buffer management, command
 * buffers). One stream per process; not reentrant, like the reference
 * (single caller thread, global state).
 */
#include "iris_internal.h"

#include <atomic>
#include <mutex>
#include <thread>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int g_init = 0;
static int g_device = -1;
static hipStream_t g_stream = nullptr;
/* side stream: launches between iris_hip_side(1) and iris_hip_side(0) go to it;
 * fork / join order it against the library stream with two events */
static hipStream_t g_side = nullptr;
static hipEvent_t g_fork_ev = nullptr, g_join_ev = nullptr;
static int g_on_side = 0;
static char g_err[512] = "";
static char g_name[256] = "";
static std::atomic<size_t> g_in_use{0};
static hipEvent_t g_events[64];
static int g_events_made = 0;
static hipGraph_t g_capture_graph = nullptr;
static int g_cus = 0;

hipStream_t iris_stream(void) { return g_on_side ? g_side : g_stream; }
int iris_cu_count(void) { return g_cus; }

int iris_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    fprintf(stderr, "iris_hip: %s\n", g_err);
    return -1;
}

int iris_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return 0;
    return iris_set_error("%s: %s", what, hipGetErrorString(e));
}

int iris_launch_check(const char *what) {
    return iris_check(hipGetLastError(), what);
}

extern "C" {

int iris_hip_init(int device) {
    if (g_init) return device < 0 || device == g_device ? 0 : iris_set_error("already bound to device %d", g_device);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return iris_set_error("no HIP device");
    if (device < 0) device = 0;
    if (device >= n) return iris_set_error("device %d of %d", device, n);
    if (iris_check(hipSetDevice(device), "hipSetDevice")) return -1;
    hipDeviceProp_t p;
    if (iris_check(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties")) return -1;
    snprintf(g_name, sizeof(g_name), "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return iris_set_error("kernels are built for gfx950, device is %s", p.gcnArchName);
    if (iris_check(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), "hipStreamCreate")) return -1;
    /* both streams at the default priority */
    if (iris_check(hipStreamCreateWithFlags(&g_side, hipStreamNonBlocking), "hipStreamCreate (side)") ||
        iris_check(hipEventCreateWithFlags(&g_fork_ev, hipEventDisableTiming), "hipEventCreate (fork)") ||
        iris_check(hipEventCreateWithFlags(&g_join_ev, hipEventDisableTiming), "hipEventCreate (join)"))
        return -1;
    g_cus = p.multiProcessorCount;
    g_device = device;
    g_init = 1;
    /* the per-kernel profile from the start (iris_print_blas_profile reports it) */
    const char *prof = getenv("IRIS_PROFILE");
    if (prof && atoi(prof) > 0) return iris_hip_profile_enable(1);
    return 0;
}

int iris_hip_available(void) {
    if (g_init) return 1;
    return iris_hip_init(0) == 0;
}

const char *iris_hip_last_error(void) { return g_err; }
const char *iris_hip_device_name(void) { return g_name; }

void *iris_hip_malloc(size_t bytes) {
    if (!iris_hip_available()) return nullptr;
    void *p = nullptr;
    size_t b = bytes ? bytes : 256;
    if (hipMalloc(&p, b) != hipSuccess) {
        iris_set_error("hipMalloc(%zu) failed", b);
        return nullptr;
    }
    g_in_use += b;
    return p;
}

void iris_hip_free(void *p) {
    if (!p) return;
    size_t sz = 0;
    if (hipMemPtrGetInfo(p, &sz) != hipSuccess) sz = 0;
    g_in_use -= sz;
    (void)hipFree(p);
}

size_t iris_hip_mem_in_use(void) { return g_in_use; }

/* Weight upload (the reference maps safetensors and copies tensor by tensor,
 * iris_safetensors.c, iris_transformer_flux.c:473-570): copies of 8 MiB and
 * more go through a ring of 4 pinned 16 MiB staging buffers. Host threads
 * copy chunk i from the (possibly mmap'd, page-faulting) source into a free
 * staging buffer while the DMA engine moves chunk i - 1 to the device, so the
 * file read, the host copy and PCIe overlap. A buffer is refilled only after
 * the event recorded behind its previous DMA has completed. The call returns
 * once the whole source has been copied out, so the caller may reuse it, as
 * with a pageable hipMemcpyAsync; during stream capture the plain copy is
 * used. */
namespace {
constexpr size_t UP_CHUNK = 16u << 20, UP_MIN = 8u << 20;
constexpr int UP_BUFS = 4, UP_THREADS = 8;
void *g_up_buf[UP_BUFS];
hipEvent_t g_up_ev[UP_BUFS];
int g_up_state;   /* 0 untried, 1 ready, -1 unavailable */
std::mutex g_up_mutex;   /* one upload at a time through the staging ring */

int up_init() {
    if (g_up_state) return g_up_state > 0 ? 0 : -1;
    g_up_state = -1;
    for (int i = 0; i < UP_BUFS; i++) {
        if (hipHostMalloc(&g_up_buf[i], UP_CHUNK, hipHostMallocDefault) != hipSuccess) return -1;
        if (hipEventCreateWithFlags(&g_up_ev[i], hipEventDisableTiming) != hipSuccess) return -1;
    }
    g_up_state = 1;
    return 0;
}

void par_memcpy(void *dst, const void *src, size_t n) {
    const size_t per = ((n + UP_THREADS - 1) / UP_THREADS + 4095) & ~(size_t)4095;
    std::thread th[UP_THREADS];
    int used = 0;
    for (size_t off = per; off < n; off += per, used++)
        th[used] = std::thread(memcpy, (char *)dst + off, (const char *)src + off, n - off < per ? n - off : per);
    memcpy(dst, src, n < per ? n : per);
    for (int i = 0; i < used; i++) th[i].join();
}

/* Small uploads (per-step inputs such as the timestep sinusoid): the source
 * is copied into one of SM_SLOTS pinned slots and the DMA reads the slot, so
 * the call returns with the source free for reuse and the copy stays
 * asynchronous; a slot is refilled only after the event behind its last copy
 * has fired. */
constexpr size_t SM_SLOT = 64u << 10;
constexpr int SM_SLOTS = 16;
char *g_sm_buf;
hipEvent_t g_sm_ev[SM_SLOTS];
int g_sm_state, g_sm_next;

int sm_init() {
    if (g_sm_state) return g_sm_state > 0 ? 0 : -1;
    g_sm_state = -1;
    if (hipHostMalloc((void **)&g_sm_buf, SM_SLOT * SM_SLOTS, hipHostMallocDefault) != hipSuccess) return -1;
    for (int i = 0; i < SM_SLOTS; i++)
        if (hipEventCreateWithFlags(&g_sm_ev[i], hipEventDisableTiming) != hipSuccess) return -1;
    g_sm_state = 1;
    return 0;
}
}  // namespace

int iris_hip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    if (!bytes) return 0;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(g_stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone;
    if (!capturing && bytes <= SM_SLOT && sm_init() == 0) {
        std::lock_guard<std::mutex> lock(g_up_mutex);
        const int b = g_sm_next;
        g_sm_next = (g_sm_next + 1) % SM_SLOTS;
        char *slot = g_sm_buf + (size_t)b * SM_SLOT;
        if (iris_check(hipEventSynchronize(g_sm_ev[b]), "small upload slot wait")) return -1;
        memcpy(slot, src, bytes);
        return iris_check(hipMemcpyAsync(dst, slot, bytes, hipMemcpyHostToDevice, g_stream), "memcpy h2d") ||
               iris_check(hipEventRecord(g_sm_ev[b], g_stream), "small upload event");
    }
    if (bytes < UP_MIN || capturing || up_init())
        return iris_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream), "memcpy h2d");
    std::lock_guard<std::mutex> lock(g_up_mutex);
    size_t i = 0;
    for (size_t off = 0; off < bytes; off += UP_CHUNK, i++) {
        const int b = (int)(i % UP_BUFS);
        const size_t n = bytes - off < UP_CHUNK ? bytes - off : UP_CHUNK;
        if (iris_check(hipEventSynchronize(g_up_ev[b]), "upload staging wait")) return -1;
        par_memcpy(g_up_buf[b], (const char *)src + off, n);
        if (iris_check(hipMemcpyAsync((char *)dst + off, g_up_buf[b], n, hipMemcpyHostToDevice, g_stream),
                       "upload chunk") ||
            iris_check(hipEventRecord(g_up_ev[b], g_stream), "upload event"))
            return -1;
    }
    return 0;
}

int iris_hip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    if (!bytes) return 0;
    if (iris_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream), "memcpy d2h")) return -1;
    return iris_check(hipStreamSynchronize(g_stream), "sync after d2h");
}

int iris_hip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    if (!bytes) return 0;
    return iris_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream), "memcpy d2d");
}

int iris_hip_memset(void *dst, int v, size_t bytes) {
    if (!bytes) return 0;
    return iris_check(hipMemsetAsync(dst, v, bytes, g_stream), "memset");
}

int iris_hip_sync(void) {
    if (!g_init) return 0;
    return iris_check(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
}

int iris_hip_event_record(int slot) {
    if (slot < 0 || slot >= 64) return iris_set_error("event slot %d", slot);
    if (!g_events_made) {
        for (int i = 0; i < 64; i++)
            if (iris_check(hipEventCreate(&g_events[i]), "hipEventCreate")) return -1;
        g_events_made = 1;
    }
    return iris_check(hipEventRecord(g_events[slot], g_stream), "hipEventRecord");
}

float iris_hip_event_elapsed_ms(int a, int b) {
    float ms = -1.0f;
    if (!g_events_made || a < 0 || b < 0 || a >= 64 || b >= 64) return -1.0f;
    if (hipEventSynchronize(g_events[b]) != hipSuccess) return -1.0f;
    if (hipEventElapsedTime(&ms, g_events[a], g_events[b]) != hipSuccess) return -1.0f;
    return ms;
}

/* ---- per-kernel profile ----
 * Each record is one launch between two events; events are created on first
 * use and reused, at most PROF_MAX launches per profile. */
}  /* extern "C" */

namespace {
constexpr int PROF_MAX = 16384;
struct ProfRec {
    const char *kernel;
    long long grid;
};
hipEvent_t g_pev[2 * PROF_MAX];
int g_pev_made;
ProfRec g_prec[PROF_MAX];
int g_prof_on, g_prof_n, g_prof_lost;
}  // namespace

int iris_prof_begin(const char *kernel, long long grid) {
    if (!g_prof_on) return -1;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g_stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return -1;
    if (g_prof_n >= PROF_MAX) {
        g_prof_lost++;
        return -1;
    }
    const int i = g_prof_n;
    while (g_pev_made < 2 * (i + 1))
        if (hipEventCreate(&g_pev[g_pev_made]) == hipSuccess) g_pev_made++;
        else return -1;
    if (hipEventRecord(g_pev[2 * i], g_stream) != hipSuccess) return -1;
    g_prec[i] = {kernel, grid};
    g_prof_n++;
    return i;
}

void iris_prof_end(int i) {
    if (i >= 0) (void)hipEventRecord(g_pev[2 * i + 1], g_stream);
}

extern "C" {

int iris_hip_profile_enable(int on) {
    if (iris_hip_sync()) return -1;
    g_prof_on = on != 0;
    g_prof_n = g_prof_lost = 0;
    return 0;
}

int iris_hip_profile_enabled(void) { return g_prof_on; }

int iris_hip_profile_read(iris_kernel_time_t *out, int max) {
    if (iris_hip_sync()) return -1;
    int n = 0;
    for (int i = 0; i < g_prof_n; i++) {
        float ms = 0.0f;
        if (iris_check(hipEventElapsedTime(&ms, g_pev[2 * i], g_pev[2 * i + 1]), "profile event")) return -1;
        int j = 0;
        while (j < n && !(out[j].grid == g_prec[i].grid && strcmp(out[j].kernel, g_prec[i].kernel) == 0)) j++;
        if (j == n) {
            if (n == max) continue;
            out[n++] = {g_prec[i].kernel, g_prec[i].grid, 0, 0.0, 1e30, 0.0};
        }
        out[j].calls++;
        out[j].total_ms += ms;
        if (ms < out[j].min_ms) out[j].min_ms = ms;
        if (ms > out[j].max_ms) out[j].max_ms = ms;
    }
    if (g_prof_lost) iris_set_error("profile: %d launches past the %d recorded", g_prof_lost, PROF_MAX);
    return n;
}

int iris_hip_fork(void) {
    if (!iris_hip_available()) return -1;
    return iris_check(hipEventRecord(g_fork_ev, g_stream), "fork record") ||
           iris_check(hipStreamWaitEvent(g_side, g_fork_ev, 0), "fork wait");
}

void iris_hip_side(int on) { g_on_side = on != 0; }

int iris_hip_join(void) {
    if (!iris_hip_available()) return -1;
    return iris_check(hipEventRecord(g_join_ev, g_side), "join record") ||
           iris_check(hipStreamWaitEvent(g_stream, g_join_ev, 0), "join wait");
}

int iris_hip_graph_begin(void) {
    if (!iris_hip_available()) return -1;
    return iris_check(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal), "begin capture");
}

void *iris_hip_graph_end(void) {
    hipGraph_t g = nullptr;
    if (iris_check(hipStreamEndCapture(g_stream, &g), "end capture")) return nullptr;
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (iris_check(e, "hipGraphInstantiate")) return nullptr;
    (void)g_capture_graph;
    return (void *)ex;
}

int iris_hip_graph_launch(void *graph) {
    return iris_check(hipGraphLaunch((hipGraphExec_t)graph, g_stream), "hipGraphLaunch");
}

void iris_hip_graph_destroy(void *graph) {
    if (graph) (void)hipGraphExecDestroy((hipGraphExec_t)graph);
}

}  /* extern "C" */
