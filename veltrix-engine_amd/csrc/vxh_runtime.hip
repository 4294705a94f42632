// Runtime part of the device C ABI: device selection, memory, copies, streams,
// events, graph capture and error reporting (include/vxh.h).
#include "vxh_internal.h"

#include <stdarg.h>
#include <string.h>

static thread_local char g_err[512] = "";
static int g_inited = 0;

extern "C" int vxh_set_error(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

extern "C" const char *vxh_last_error(void) { return g_err; }

extern "C" int vxh_init(void)
{
    if (g_inited) return VXH_OK;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1)
        return vxh_fail(VXH_ERR_NODEVICE, "no HIP device visible (%s)",
                        e == hipSuccess ? "count 0" : hipGetErrorString(e));
    VXH_CHECK(hipSetDevice(0));
    hipDeviceProp_t prop;
    VXH_CHECK(hipGetDeviceProperties(&prop, 0));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return vxh_fail(VXH_ERR_UNSUPPORTED, "device is %s; the library's kernels are compiled for gfx950 only",
                        prop.gcnArchName);
    g_inited = 1;
    return VXH_OK;
}

extern "C" int vxh_device_name(char *buf, int len)
{
    int rc = vxh_init();
    if (rc) return rc;
    hipDeviceProp_t prop;
    VXH_CHECK(hipGetDeviceProperties(&prop, 0));
    snprintf(buf, (size_t)len, "%s (%s, %d CUs)", prop.name, prop.gcnArchName,
             prop.multiProcessorCount);
    return VXH_OK;
}

extern "C" int vxh_malloc(void **p, size_t bytes)
{
    int rc = vxh_init();
    if (rc) return rc;
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess)
        return vxh_fail(VXH_ERR_ALLOC, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return VXH_OK;
}

extern "C" int vxh_free(void *p)
{
    if (!p) return VXH_OK;
    VXH_CHECK(hipFree(p));
    return VXH_OK;
}

extern "C" int vxh_upload(void *dst, const void *src, size_t bytes, vxh_stream s)
{
    if (!bytes) return VXH_OK;
    VXH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, vxh_hs(s)));
    VXH_CHECK(hipStreamSynchronize(vxh_hs(s)));
    return VXH_OK;
}

extern "C" int vxh_host_alloc(void **p, size_t bytes)
{
    int rc = vxh_init();
    if (rc) return rc;
    *p = nullptr;
    if (bytes == 0) bytes = 64;
    hipError_t e = hipHostMalloc(p, bytes, hipHostMallocDefault);
    if (e != hipSuccess)
        return vxh_fail(VXH_ERR_ALLOC, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return VXH_OK;
}

extern "C" int vxh_host_free(void *p)
{
    if (!p) return VXH_OK;
    VXH_CHECK(hipHostFree(p));
    return VXH_OK;
}

extern "C" int vxh_upload_async(void *dst, const void *src, size_t bytes, vxh_stream s)
{
    if (!bytes) return VXH_OK;
    VXH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, vxh_hs(s)));
    return VXH_OK;
}

extern "C" int vxh_download(void *dst, const void *src, size_t bytes, vxh_stream s)
{
    if (!bytes) return VXH_OK;
    VXH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, vxh_hs(s)));
    VXH_CHECK(hipStreamSynchronize(vxh_hs(s)));
    return VXH_OK;
}

extern "C" int vxh_copy(void *dst, const void *src, size_t bytes, vxh_stream s)
{
    if (!bytes) return VXH_OK;
    VXH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, vxh_hs(s)));
    return VXH_OK;
}

__global__ void vx_fill_f32_kernel(float *__restrict__ p, float v, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
}

extern "C" int vxh_fill_f32(float *dst, float value, size_t n, vxh_stream s)
{
    if (!n) return VXH_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    vx_fill_f32_kernel<<<(unsigned)blocks, 256, 0, vxh_hs(s)>>>(dst, value, n);
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" int vxh_stream_create(vxh_stream *s)
{
    int rc = vxh_init();
    if (rc) return rc;
    hipStream_t h;
    VXH_CHECK(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
    *s = (vxh_stream)h;
    return VXH_OK;
}

extern "C" int vxh_stream_destroy(vxh_stream s)
{
    if (s) VXH_CHECK(hipStreamDestroy(vxh_hs(s)));
    return VXH_OK;
}

extern "C" int vxh_stream_sync(vxh_stream s)
{
    VXH_CHECK(hipStreamSynchronize(vxh_hs(s)));
    return VXH_OK;
}

extern "C" int vxh_device_sync(void)
{
    int rc = vxh_init();
    if (rc) return rc;
    VXH_CHECK(hipDeviceSynchronize());
    return VXH_OK;
}

extern "C" int vxh_event_create(vxh_event *e)
{
    int rc = vxh_init();
    if (rc) return rc;
    hipEvent_t h;
    VXH_CHECK(hipEventCreate(&h));
    *e = (vxh_event)h;
    return VXH_OK;
}

extern "C" int vxh_event_destroy(vxh_event e)
{
    if (e) VXH_CHECK(hipEventDestroy((hipEvent_t)e));
    return VXH_OK;
}

extern "C" int vxh_event_record(vxh_event e, vxh_stream s)
{
    VXH_CHECK(hipEventRecord((hipEvent_t)e, vxh_hs(s)));
    return VXH_OK;
}

extern "C" int vxh_event_elapsed_ms(vxh_event a, vxh_event b, float *ms)
{
    VXH_CHECK(hipEventSynchronize((hipEvent_t)b));
    VXH_CHECK(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return VXH_OK;
}

struct vxh_graph_s {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

extern "C" int vxh_capture_begin(vxh_stream s)
{
    VXH_CHECK(hipStreamBeginCapture(vxh_hs(s), hipStreamCaptureModeThreadLocal));
    return VXH_OK;
}

extern "C" int vxh_capture_end(vxh_stream s, vxh_graph *g)
{
    hipGraph_t graph;
    VXH_CHECK(hipStreamEndCapture(vxh_hs(s), &graph));
    hipGraphExec_t exec;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return vxh_fail(VXH_ERR_LAUNCH, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    vxh_graph_s *r = new vxh_graph_s{graph, exec};
    *g = r;
    return VXH_OK;
}

extern "C" int vxh_graph_launch(vxh_graph g, vxh_stream s)
{
    VXH_CHECK(hipGraphLaunch(g->exec, vxh_hs(s)));
    return VXH_OK;
}

extern "C" int vxh_graph_destroy(vxh_graph g)
{
    if (!g) return VXH_OK;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
    return VXH_OK;
}

extern "C" int vxh_workspace_alloc(vxh_workspace *w, size_t acc_elems, size_t part_floats)
{
    memset(w, 0, sizeof(*w));
    int rc = vxh_malloc((void **)&w->acc, acc_elems * sizeof(double));
    if (rc) return rc;
    rc = vxh_malloc((void **)&w->part, part_floats * sizeof(float));
    if (rc) { vxh_free(w->acc); w->acc = nullptr; return rc; }
    // the accumulator starts zeroed; every consumer clears what it reads
    VXH_CHECK(hipMemset(w->acc, 0, acc_elems * sizeof(double)));
    VXH_CHECK(hipDeviceSynchronize());
    w->acc_elems = acc_elems;
    w->part_floats = part_floats;
    return VXH_OK;
}

extern "C" int vxh_workspace_free(vxh_workspace *w)
{
    vxh_free(w->acc);
    vxh_free(w->part);
    memset(w, 0, sizeof(*w));
    return VXH_OK;
}
