// ti_runtime.hip — context, buffers, events and graph capture for libtabinfer.
// Replaces the reference's WebGPU core (engine/webgpu-engine.js): one HIP
// stream per context is the FIFO queue, a captured hipGraph is the
// "one command encoder per decode step" batch, hipEvents are the timestamps.
#include "ti_internal.h"
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <stdlib.h>

int ti_hip_fail(hipError_t e, const char* what) {
    int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? TI_ERR_OOM
             : (e == hipErrorNoDevice || e == hipErrorInvalidDevice) ? TI_ERR_NO_DEVICE : TI_ERR_HIP;
    return ti_fail(code, "%s: %s", what, hipGetErrorString(e));
}

extern "C" int ti_version(void) { return 100; }

extern "C" int ti_device_count(int* n) {
    TI_REQUIRE(n, "ti_device_count: null output");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if (e == hipErrorNoDevice) { *n = 0; return TI_OK; }
    if (e != hipSuccess) { *n = 0; return ti_hip_fail(e, "hipGetDeviceCount"); }
    *n = c;
    return TI_OK;
}

// Releases everything a (possibly partly built) context holds: scratch, the 64 events,
// the stream, the host struct. Used by ti_shutdown and by every ti_init error path.
static void destroy_ctx(ti_ctx* c) {
    void* ps[] = {c->act_q, c->act_s, c->act_sum, c->attn_po, c->attn_ml, c->amax_v, c->amax_i,
                  c->moe_cnt, c->moe_off, c->moe_fill, c->moe_sidx, c->tg_part, c->qkv_pub, c->sync};
    for (void* p : ps) if (p) (void)hipFree(p);
    for (int i = 0; i < 64; i++) if (c->ev[i]) (void)hipEventDestroy(c->ev[i]);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    free(c);
}

extern "C" int ti_init(int device, ti_ctx** out) {
    TI_REQUIRE(out, "ti_init: null output");
    *out = nullptr;
    int n = 0;
    int rc = ti_device_count(&n);
    if (rc) return rc;
    if (n == 0) return ti_fail(TI_ERR_NO_DEVICE, "ti_init: no HIP device visible");
    if (device < 0 || device >= n) return ti_fail(TI_ERR_NO_DEVICE, "ti_init: device %d out of range (have %d)", device, n);
    hipDeviceProp_t prop;
    TI_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return ti_fail(TI_ERR_NO_DEVICE, "ti_init: device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    TI_HIP(hipSetDevice(device));
    ti_ctx* c = (ti_ctx*)calloc(1, sizeof(ti_ctx));
    if (!c) return ti_fail(TI_ERR_OOM, "ti_init: host allocation failed");
    c->device = device;
    c->cus = prop.multiProcessorCount;
    {
        const char* sep = getenv("TI_DECODE_QKV_SEPARATE");
        c->qkv_separate = sep && *sep && strcmp(sep, "0") != 0;
        const char* polls = getenv("TI_DECODE_QKV_POLLS");
        c->qkv_polls = polls && *polls ? atoi(polls) : -1;   // -1: the kernel's own bound
    }
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) { c->stream = nullptr; destroy_ctx(c); return ti_hip_fail(e, "hipStreamCreateWithFlags"); }
    for (int i = 0; i < 64; i++) {
        e = hipEventCreate(&c->ev[i]);
        if (e != hipSuccess) { c->ev[i] = nullptr; destroy_ctx(c); return ti_hip_fail(e, "hipEventCreate"); }
    }
    struct { void** p; size_t bytes; } allocs[] = {
        {(void**)&c->act_q, (size_t)TI_ACT_CAP * TI_ACT_TMAX},
        {(void**)&c->act_s, (size_t)TI_ACT_CAP / 32 * TI_ACT_TMAX * 4},
        {(void**)&c->act_sum, (size_t)TI_ACT_CAP / 16 * 4},
        {(void**)&c->attn_po, (size_t)TI_ATTN_ROWSPLITS * TI_ATTN_HD_MAX * 4},
        {(void**)&c->attn_ml, (size_t)TI_ATTN_ROWSPLITS * 2 * 4},
        {(void**)&c->amax_v, (size_t)TI_AMAX_PARTS * 4},
        {(void**)&c->amax_i, (size_t)TI_AMAX_PARTS * 4},
        {(void**)&c->moe_cnt, (size_t)TI_MOE_E_MAX * 4},
        {(void**)&c->moe_off, (size_t)(TI_MOE_E_MAX + 1) * 4},
        {(void**)&c->moe_fill, (size_t)TI_MOE_E_MAX * 4},
        {(void**)&c->moe_sidx, (size_t)TI_MOE_P_MAX * 4},
        {(void**)&c->tg_part, (size_t)TI_TG_SPLIT_BLOCKS * 2 * 256 * 4},
        {(void**)&c->qkv_pub, (size_t)TI_QKV_PUB_WORDS * 8},
        {(void**)&c->sync, (size_t)TI_SYNC_WORDS * 4},
    };
    for (auto& a : allocs) {
        e = hipMalloc(a.p, a.bytes);
        if (e != hipSuccess) { destroy_ctx(c); return ti_hip_fail(e, "ti_init scratch hipMalloc"); }
    }
    e = hipMemset(c->moe_cnt, 0, TI_MOE_E_MAX * 4);
    if (e == hipSuccess) e = hipMemset(c->sync, 0, TI_SYNC_WORDS * 4);
    if (e == hipSuccess) e = hipMemset(c->qkv_pub, 0, (size_t)TI_QKV_PUB_WORDS * 8);   // epoch 0: never current
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) { destroy_ctx(c); return ti_hip_fail(e, "ti_init scratch clear"); }
    *out = c;
    return TI_OK;
}

extern "C" int ti_shutdown(ti_ctx* c) {
    TI_CHECK_CTX(c);
    TI_HIP(hipSetDevice(c->device));
    (void)hipStreamSynchronize(c->stream);
    destroy_ctx(c);
    return TI_OK;
}

extern "C" int ti_buf_alloc(ti_ctx* c, size_t bytes, void** dptr) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(dptr, "ti_buf_alloc: null output");
    TI_REQUIRE(!c->capturing, "ti_buf_alloc: not allowed while a graph is being captured");
    *dptr = nullptr;
    TI_HIP(hipSetDevice(c->device));
    TI_HIP(hipMalloc(dptr, bytes ? bytes : 1));
    return TI_OK;
}

extern "C" int ti_buf_free(ti_ctx* c, void* dptr) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(!c->capturing, "ti_buf_free: not allowed while a graph is being captured");
    if (!dptr) return TI_OK;
    TI_HIP(hipSetDevice(c->device));
    TI_HIP(hipStreamSynchronize(c->stream));   // deferred-destroy semantics: in-flight work finishes first
    TI_HIP(hipFree(dptr));
    return TI_OK;
}

extern "C" int ti_buf_write(ti_ctx* c, void* dst, size_t off, const void* src, size_t bytes) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(dst && (src || !bytes), "ti_buf_write: null pointer");
    TI_REQUIRE(!c->capturing, "ti_buf_write: host copies cannot be captured");
    if (!bytes) return TI_OK;
    TI_HIP(hipSetDevice(c->device));
    TI_HIP(hipMemcpyAsync((char*)dst + off, src, bytes, hipMemcpyHostToDevice, c->stream));
    TI_HIP(hipStreamSynchronize(c->stream));
    return TI_OK;
}

extern "C" int ti_buf_read(ti_ctx* c, const void* src, size_t off, void* dst, size_t bytes) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(src && (dst || !bytes), "ti_buf_read: null pointer");
    TI_REQUIRE(!c->capturing, "ti_buf_read: host copies cannot be captured");
    if (!bytes) return TI_OK;
    TI_HIP(hipSetDevice(c->device));
    TI_HIP(hipMemcpyAsync(dst, (const char*)src + off, bytes, hipMemcpyDeviceToHost, c->stream));
    TI_HIP(hipStreamSynchronize(c->stream));
    return TI_OK;
}

// Stream-ordered device -> host copy that does not wait: complete once the work issued
// before it is (ti_event_record after it, then ti_event_wait). dst should be pinned
// (ti_host_alloc) for the copy to run asynchronously.
extern "C" int ti_buf_read_async(ti_ctx* c, const void* src, size_t off, void* dst, size_t bytes) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(src && dst, "ti_buf_read_async: null buffer");
    TI_REQUIRE(!c->capturing, "ti_buf_read_async: not during graph capture");
    if (!bytes) return TI_OK;
    TI_HIP(hipMemcpyAsync(dst, static_cast<const char*>(src) + off, bytes, hipMemcpyDeviceToHost, c->stream));
    return TI_OK;
}

// page-locked host memory (hipHostMalloc), the target of asynchronous reads
extern "C" int ti_host_alloc(size_t bytes, void** out) {
    TI_REQUIRE(out && bytes > 0, "ti_host_alloc: need bytes > 0 and an output pointer");
    *out = nullptr;
    TI_HIP(hipHostMalloc(out, bytes, hipHostMallocDefault));
    return TI_OK;
}

// frees ti_host_alloc memory after the device has finished every queued operation, so a
// copy still in flight into the memory never lands in freed pages
extern "C" int ti_host_free(void* p) {
    if (!p) return TI_OK;
    TI_HIP(hipDeviceSynchronize());
    TI_HIP(hipHostFree(p));
    return TI_OK;
}

// Device-to-device copy as a plain streaming kernel (one read and one write of every
// byte; graph-capturable): it is also the known-size reference that scales the HBM
// byte counters of the other kernels.
__global__ __launch_bounds__(256) void k_copy_u4(const uint4* __restrict__ s, uint4* __restrict__ d, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) d[i] = s[i];
}
__global__ __launch_bounds__(256) void k_copy_u8(const uint8_t* __restrict__ s, uint8_t* __restrict__ d, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) d[i] = s[i];
}

extern "C" int ti_buf_copy(ti_ctx* c, void* dst, size_t doff, const void* src, size_t soff, size_t bytes) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(dst && src, "ti_buf_copy: null pointer");
    if (!bytes) return TI_OK;
    TI_HIP(hipSetDevice(c->device));
    const char* s = (const char*)src + soff;
    char* d = (char*)dst + doff;
    TI_REQUIRE(s + bytes <= d || d + bytes <= s || s == d, "ti_buf_copy: overlapping ranges");
    if ((((uintptr_t)s | (uintptr_t)d | bytes) & 15u) == 0) {
        const size_t n16 = bytes / 16;
        size_t blocks = (n16 + 255) / 256;
        blocks = blocks < 8192 ? blocks : 8192;
        k_copy_u4<<<(unsigned)blocks, 256, 0, c->stream>>>(reinterpret_cast<const uint4*>(s), reinterpret_cast<uint4*>(d), n16);
    } else {
        size_t blocks = (bytes + 255) / 256;
        blocks = blocks < 8192 ? blocks : 8192;
        k_copy_u8<<<(unsigned)blocks, 256, 0, c->stream>>>(reinterpret_cast<const uint8_t*>(s), reinterpret_cast<uint8_t*>(d), bytes);
    }
    TI_LAUNCHED("k_copy");
    return TI_OK;
}

__global__ void k_fill_u32(uint32_t* __restrict__ p, uint32_t v, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
}

int ti_fill_u32_async(ti_ctx* c, void* dst, uint32_t value, size_t count) {
    if (!count) return TI_OK;
    size_t blocks = (count + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    k_fill_u32<<<(unsigned)blocks, 256, 0, c->stream>>>((uint32_t*)dst, value, count);
    TI_LAUNCHED("k_fill_u32");
    return TI_OK;
}

extern "C" int ti_buf_fill_u32(ti_ctx* c, void* dst, uint32_t value, size_t count) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(dst, "ti_buf_fill_u32: null pointer");
    return ti_fill_u32_async(c, dst, value, count);
}

extern "C" int ti_sync(ti_ctx* c) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(!c->capturing, "ti_sync: cannot wait inside graph capture");
    TI_HIP(hipStreamSynchronize(c->stream));
    return TI_OK;
}

extern "C" int ti_event_record(ti_ctx* c, int slot) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(slot >= 0 && slot < 64, "ti_event_record: slot %d out of [0,64)", slot);
    // inside a capture the record becomes an event-record node of the graph (an external
    // event), so every replay timestamps the point where it sits between the kernels
    if (c->capturing) TI_HIP(hipEventRecordWithFlags(c->ev[slot], c->stream, hipEventRecordExternal));
    else TI_HIP(hipEventRecord(c->ev[slot], c->stream));
    return TI_OK;
}

// Waits for the last record of one slot (not the whole stream), so a host can consume an
// early batch while later ones run. May run on another thread than the context's owner,
// provided nothing re-records the slot until it returns.
extern "C" int ti_event_wait(ti_ctx* c, int slot) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(slot >= 0 && slot < 64, "ti_event_wait: slot %d out of [0,64)", slot);
    TI_HIP(hipEventSynchronize(c->ev[slot]));
    return TI_OK;
}

extern "C" int ti_event_elapsed_ms(ti_ctx* c, int a, int b, float* ms) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(a >= 0 && a < 64 && b >= 0 && b < 64 && ms, "ti_event_elapsed_ms: bad arguments");
    TI_HIP(hipEventSynchronize(c->ev[b]));
    TI_HIP(hipEventElapsedTime(ms, c->ev[a], c->ev[b]));
    return TI_OK;
}

extern "C" int ti_graph_begin(ti_ctx* c) {
    TI_CHECK_CTX(c);
    if (c->capturing) return ti_fail(TI_ERR_STATE, "ti_graph_begin: capture already open");
    TI_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = 1;
    return TI_OK;
}

extern "C" int ti_graph_end(ti_ctx* c, ti_graph** out) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(out, "ti_graph_end: null output");
    *out = nullptr;
    if (!c->capturing) return ti_fail(TI_ERR_STATE, "ti_graph_end: no capture open");
    c->capturing = 0;
    hipGraph_t g = nullptr;
    TI_HIP(hipStreamEndCapture(c->stream, &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) { (void)hipGraphDestroy(g); return ti_hip_fail(e, "hipGraphInstantiate"); }
    ti_graph* tg = (ti_graph*)calloc(1, sizeof(ti_graph));
    if (!tg) { (void)hipGraphExecDestroy(ex); (void)hipGraphDestroy(g); return ti_fail(TI_ERR_OOM, "ti_graph_end: host alloc"); }
    tg->graph = g;
    tg->exec = ex;
    tg->device = c->device;
    *out = tg;
    return TI_OK;
}

extern "C" int ti_graph_launch(ti_ctx* c, ti_graph* g) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(g, "ti_graph_launch: null graph");
    TI_REQUIRE(!c->capturing, "ti_graph_launch: cannot launch a graph inside a capture");
    TI_HIP(hipGraphLaunch(g->exec, c->stream));
    return TI_OK;
}

extern "C" int ti_graph_destroy(ti_graph* g) {
    if (!g) return TI_OK;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    free(g);
    return TI_OK;
}
