// Host runtime of liblcdhip.so: context, buffers, streams, run-time
// compilation (hiprtc), module launch, the wavefront level loop, hipGraph
// capture, and a few utility kernels (fill, digest, diagonal lookup, machine
// constant probes).  Replaces compiler/cuda_runtime.py and the device-facing
// half of compiler/scheduler.py of the reference.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "lcdhip_common.h"

namespace lcdhip {

static thread_local std::string g_error;

void set_error(const char *format, ...)
{
    char buffer[2048];
    va_list args;
    va_start(args, format);
    vsnprintf(buffer, sizeof(buffer), format, args);
    va_end(args);
    g_error = buffer;
}

Context &context()
{
    static Context ctx;
    return ctx;
}

bool initialised() { return context().ready; }

hipStream_t resolve_stream(lcdhip_stream stream)
{
    return stream ? reinterpret_cast<hipStream_t>(stream) : context().stream;
}

}  // namespace lcdhip

using lcdhip::context;
using lcdhip::resolve_stream;
using lcdhip::set_error;

struct lcdhip_module {
    hipModule_t module = nullptr;
};
struct lcdhip_kernel {
    hipFunction_t function = nullptr;
};
struct lcdhip_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

extern "C" const char *lcdhip_last_error(void) { return lcdhip::g_error.c_str(); }

extern "C" const char *lcdhip_version(void)
{
    // (with the version of the run-time compiler: what a code object that is
    // kept between processes has to be keyed by)
    static char text[96];
    int major = 0, minor = 0;
    if (hiprtcVersion(&major, &minor) != HIPRTC_SUCCESS) major = minor = 0;
    snprintf(text, sizeof(text), "lcdhip 0.2 (gfx950; hiprtc %d.%d; HIP %d.%d.%d)", major, minor,
             HIP_VERSION_MAJOR, HIP_VERSION_MINOR, HIP_VERSION_PATCH);
    return text;
}

extern "C" int lcdhip_device_count(int *count)
{
    if (!count) {
        set_error("count is NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    *count = 0;
    hipError_t status = hipGetDeviceCount(count);
    if (status != hipSuccess) {
        *count = 0;
        set_error("hipGetDeviceCount: %s", hipGetErrorString(status));
        return LCDHIP_ERR_NO_DEVICE;
    }
    return LCDHIP_OK;
}

// Work area of lcdhip_digest_noalloc: the per-workgroup partial results of
// the digest kernels (16 KiB).  One copy per GPU, held until the process
// ends.  The array's name is only a host-side handle; its address on a device
// comes from hipGetSymbolAddress while that device is current (lcdhip_init)
// and is what host code passes on.
#define LCDHIP_DIGEST_SCRATCH_WORDS (2 * 1024)
static __device__ __align__(256) unsigned long long
    lcdhip_digest_scratch[LCDHIP_DIGEST_SCRATCH_WORDS];
#define LCDHIP_MAX_DEVICES 64
static unsigned long long *g_digest_scratch[LCDHIP_MAX_DEVICES] = {};

// ---------------------------------------------------- block pool ----
namespace lcdhip {
namespace {
struct Pool {
    std::mutex lock;
    std::unordered_map<void *, std::pair<size_t, int>> blocks;   // capacity, device
    std::multimap<std::pair<int, size_t>, void *> idle;          // (device, capacity)
    size_t idle_bytes = 0;
};
Pool &pool()
{
    static Pool instance;
    return instance;
}
size_t pool_capacity(size_t bytes)
{
    // powers of two up to 1 MiB, multiples of 1 MiB beyond
    if (bytes <= 256)
        return 256;
    if (bytes > (size_t(1) << 20))
        return (bytes + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    size_t capacity = 256;
    while (capacity < bytes)
        capacity <<= 1;
    return capacity;
}
}  // namespace

hipError_t pool_alloc(void **out, size_t bytes)
{
    *out = nullptr;
    int device = 0;
    hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess)
        return status;
    const size_t capacity = pool_capacity(bytes);
    Pool &p = pool();
    {
        std::lock_guard<std::mutex> guard(p.lock);
        auto found = p.idle.find({device, capacity});
        if (found != p.idle.end()) {
            *out = found->second;
            p.idle.erase(found);
            p.idle_bytes -= capacity;
            return hipSuccess;
        }
    }
    void *pointer = nullptr;
    status = hipMalloc(&pointer, capacity);
    if (status != hipSuccess) {
        // what is idle may be what is missing
        pool_trim();
        status = hipMalloc(&pointer, capacity);
        if (status != hipSuccess)
            return status;
    }
    std::lock_guard<std::mutex> guard(p.lock);
    p.blocks[pointer] = {capacity, device};
    *out = pointer;
    return hipSuccess;
}

void pool_release(void *pointer)
{
    if (!pointer)
        return;
    Pool &p = pool();
    std::unique_lock<std::mutex> guard(p.lock);
    auto found = p.blocks.find(pointer);
    if (found == p.blocks.end()) {
        guard.unlock();
        (void)hipFree(pointer);
        return;
    }
    const size_t capacity = found->second.first;
    if (capacity > kPoolIdleBytes) {
        p.blocks.erase(found);
        guard.unlock();
        (void)hipFree(pointer);
        return;
    }
    // what comes back is what the next call will ask for: make room for it
    // by freeing blocks that have been idle (of other sizes: an earlier
    // structure's) rather than the one just used
    std::vector<void *> evicted;
    while (p.idle_bytes + capacity > kPoolIdleBytes && !p.idle.empty()) {
        auto victim = p.idle.begin();
        if (victim->first.second == capacity && p.idle.size() > 1)
            victim = std::prev(p.idle.end());
        p.idle_bytes -= victim->first.second;
        evicted.push_back(victim->second);
        p.blocks.erase(victim->second);
        p.idle.erase(victim);
    }
    p.idle.insert({{found->second.second, capacity}, pointer});
    p.idle_bytes += capacity;
    guard.unlock();
    for (void *old : evicted)
        (void)hipFree(old);
}

namespace {
std::atomic<int> g_open_captures{0};
}

void pool_retire(void *const *pointers, size_t count)
{
    bool any = false;
    for (size_t k = 0; k < count; ++k)
        any = any || pointers[k] != nullptr;
    if (!any)
        return;
    if (g_open_captures.load() > 0) {
        Pool &p = pool();
        for (size_t k = 0; k < count; ++k) {
            if (!pointers[k])
                continue;
            {
                std::lock_guard<std::mutex> guard(p.lock);
                p.blocks.erase(pointers[k]);
            }
            (void)hipFree(pointers[k]);
        }
        return;
    }
    (void)hipDeviceSynchronize();
    for (size_t k = 0; k < count; ++k)
        pool_release(pointers[k]);
}

void pool_trim()
{
    Pool &p = pool();
    std::vector<void *> doomed;
    {
        std::lock_guard<std::mutex> guard(p.lock);
        for (auto &entry : p.idle) {
            doomed.push_back(entry.second);
            p.blocks.erase(entry.second);
        }
        p.idle.clear();
        p.idle_bytes = 0;
    }
    for (void *pointer : doomed)
        (void)hipFree(pointer);
}
}  // namespace lcdhip

extern "C" int lcdhip_init(int device)
{
    auto &ctx = context();
    if (ctx.ready && ctx.device == device)
        return LCDHIP_OK;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        set_error("no HIP device is visible; liblcdhip needs an MI355X-class GPU");
        return LCDHIP_ERR_NO_DEVICE;
    }
    if (device < 0 || device >= count) {
        set_error("device %d out of range (found %d)", device, count);
        return LCDHIP_ERR_ARGUMENT;
    }
    LCDHIP_CHECK(hipSetDevice(device));
    LCDHIP_CHECK(hipGetDeviceProperties(&ctx.props, device));
    if (ctx.stream == nullptr)
        LCDHIP_CHECK(hipStreamCreateWithFlags(&ctx.stream, hipStreamNonBlocking));
    if (device < LCDHIP_MAX_DEVICES && g_digest_scratch[device] == nullptr) {
        void *address = nullptr;
        LCDHIP_CHECK(hipGetSymbolAddress(&address,
                                         HIP_SYMBOL(lcdhip_digest_scratch)));
        g_digest_scratch[device] = static_cast<unsigned long long *>(address);
    }
    ctx.device = device;
    ctx.ready = true;
    return LCDHIP_OK;
}

extern "C" int lcdhip_shutdown(void)
{
    auto &ctx = context();
    if (!ctx.ready)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipStreamSynchronize(ctx.stream));
    lcdhip::pool_trim();
    LCDHIP_CHECK(hipStreamDestroy(ctx.stream));
    ctx.stream = nullptr;
    ctx.ready = false;
    ctx.device = -1;
    return LCDHIP_OK;
}

extern "C" int lcdhip_device_props(lcdhip_props *out)
{
    LCDHIP_REQUIRE_INIT();
    if (!out) {
        set_error("out is NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    const hipDeviceProp_t &p = context().props;
    memset(out, 0, sizeof(*out));
    out->compute_units = p.multiProcessorCount;
    // gfx942/gfx950 parts group their CUs into XCDs of 32 (some fused off).
    out->xcd_count = std::max(1, (p.multiProcessorCount + 37) / 38);
    out->wavefront_size = p.warpSize;
    out->max_threads_per_block = p.maxThreadsPerBlock;
    out->lds_bytes_per_block = static_cast<int32_t>(p.sharedMemPerBlock);
    out->lds_bytes_per_cu = static_cast<int32_t>(p.maxSharedMemoryPerMultiProcessor);
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bus_bits = p.memoryBusWidth;
    out->l2_bytes = p.l2CacheSize;
    out->global_memory_bytes = static_cast<int64_t>(p.totalGlobalMem);
    snprintf(out->name, sizeof(out->name), "%s", p.name);
    snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
    return LCDHIP_OK;
}

// ------------------------------------------------------------ buffers ----

extern "C" int lcdhip_buffer_alloc(size_t bytes, void **d_out)
{
    LCDHIP_REQUIRE_INIT();
    if (!d_out) {
        set_error("d_out is NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    *d_out = nullptr;
    LCDHIP_CHECK(hipMalloc(d_out, bytes ? bytes : 4));
    return LCDHIP_OK;
}

extern "C" int lcdhip_buffer_free(void *d_ptr)
{
    if (!d_ptr)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipFree(d_ptr));
    return LCDHIP_OK;
}

extern "C" int lcdhip_buffer_upload(void *d_dst, const void *host_src,
                                    size_t bytes, lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (bytes == 0)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipMemcpyAsync(d_dst, host_src, bytes, hipMemcpyHostToDevice,
                                resolve_stream(stream)));
    return LCDHIP_OK;
}

extern "C" int lcdhip_buffer_download(void *host_dst, const void *d_src,
                                      size_t bytes, lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (bytes == 0)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipMemcpyAsync(host_dst, d_src, bytes, hipMemcpyDeviceToHost,
                                resolve_stream(stream)));
    return LCDHIP_OK;
}

extern "C" int lcdhip_buffer_copy(void *d_dst, const void *d_src, size_t bytes,
                                  lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (bytes == 0)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice,
                                resolve_stream(stream)));
    return LCDHIP_OK;
}

__global__ void lcdhip_fill32_kernel(uint32_t *dst, uint32_t value, size_t count)
{
    size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (; i < count; i += stride)
        dst[i] = value;
}

extern "C" int lcdhip_buffer_fill32(void *d_dst, uint32_t value, size_t count,
                                    lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (count == 0)
        return LCDHIP_OK;
    unsigned blocks = static_cast<unsigned>(
        std::min<size_t>((count + 255) / 256, 16384));
    hipLaunchKernelGGL(lcdhip_fill32_kernel, dim3(blocks), dim3(256), 0,
                       resolve_stream(stream), static_cast<uint32_t *>(d_dst),
                       value, count);
    LCDHIP_CHECK(hipGetLastError());
    return LCDHIP_OK;
}

extern "C" int lcdhip_host_alloc(size_t bytes, void **host_out)
{
    LCDHIP_REQUIRE_INIT();
    if (!host_out) {
        set_error("host_out is NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    LCDHIP_CHECK(hipHostMalloc(host_out, bytes ? bytes : 4, hipHostMallocDefault));
    return LCDHIP_OK;
}

extern "C" int lcdhip_host_free(void *host_ptr)
{
    if (!host_ptr)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipHostFree(host_ptr));
    return LCDHIP_OK;
}

extern "C" int lcdhip_stream_create(lcdhip_stream *out)
{
    LCDHIP_REQUIRE_INIT();
    hipStream_t stream = nullptr;
    LCDHIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    *out = stream;
    return LCDHIP_OK;
}

extern "C" int lcdhip_stream_destroy(lcdhip_stream stream)
{
    if (!stream)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipStreamDestroy(reinterpret_cast<hipStream_t>(stream)));
    return LCDHIP_OK;
}

extern "C" int lcdhip_stream_sync(lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    LCDHIP_CHECK(hipStreamSynchronize(resolve_stream(stream)));
    return LCDHIP_OK;
}

extern "C" int lcdhip_event_create(lcdhip_event *out)
{
    LCDHIP_REQUIRE_INIT();
    hipEvent_t event = nullptr;
    LCDHIP_CHECK(hipEventCreate(&event));
    *out = event;
    return LCDHIP_OK;
}

extern "C" int lcdhip_event_destroy(lcdhip_event event)
{
    if (!event)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    return LCDHIP_OK;
}

extern "C" int lcdhip_event_record(lcdhip_event event, lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    LCDHIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(event),
                                resolve_stream(stream)));
    return LCDHIP_OK;
}

extern "C" int lcdhip_event_elapsed_ms(lcdhip_event start, lcdhip_event stop,
                                       float *ms)
{
    LCDHIP_REQUIRE_INIT();
    LCDHIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
    LCDHIP_CHECK(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                     reinterpret_cast<hipEvent_t>(stop)));
    return LCDHIP_OK;
}

// ------------------------------------------------------------ modules ----

extern "C" void lcdhip_free_host(void *ptr) { free(ptr); }

extern "C" int lcdhip_module_compile_code(const char *source, const char *name,
                                          const char *const *options,
                                          int option_count, void **code_out,
                                          size_t *size_out, char **log_out)
{
    if (!source || !code_out || !size_out) {
        set_error("source/code_out/size_out must not be NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    *code_out = nullptr;
    *size_out = 0;
    if (log_out)
        *log_out = nullptr;
    hiprtcProgram program = nullptr;
    hiprtcResult result = hiprtcCreateProgram(
        &program, source, name ? name : "lcd_generated.hip", 0, nullptr, nullptr);
    if (result != HIPRTC_SUCCESS) {
        set_error("hiprtcCreateProgram: %s", hiprtcGetErrorString(result));
        return LCDHIP_ERR_COMPILE;
    }
    std::vector<const char *> opts(options, options + option_count);
    result = hiprtcCompileProgram(program, static_cast<int>(opts.size()),
                                  opts.data());
    size_t log_size = 0;
    hiprtcGetProgramLogSize(program, &log_size);
    std::string log(log_size, '\0');
    if (log_size)
        hiprtcGetProgramLog(program, log.data());
    if (log_out) {
        *log_out = static_cast<char *>(malloc(log.size() + 1));
        memcpy(*log_out, log.c_str(), log.size() + 1);
    }
    if (result != HIPRTC_SUCCESS) {
        set_error("hiprtc: %s\n%s", hiprtcGetErrorString(result), log.c_str());
        hiprtcDestroyProgram(&program);
        return LCDHIP_ERR_COMPILE;
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(program, &code_size);
    void *code = malloc(code_size ? code_size : 1);
    hiprtcGetCode(program, static_cast<char *>(code));
    hiprtcDestroyProgram(&program);
    *code_out = code;
    *size_out = code_size;
    return LCDHIP_OK;
}

extern "C" int lcdhip_module_load(const void *code, size_t size,
                                  lcdhip_module **out)
{
    LCDHIP_REQUIRE_INIT();
    if (!code || !size || !out) {
        set_error("code/out must not be NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    auto *module = new lcdhip_module();
    hipError_t status = hipModuleLoadData(&module->module, code);
    if (status != hipSuccess) {
        set_error("hipModuleLoadData: %s", hipGetErrorString(status));
        delete module;
        return LCDHIP_ERR_HIP;
    }
    *out = module;
    return LCDHIP_OK;
}

extern "C" int lcdhip_module_destroy(lcdhip_module *module)
{
    if (!module)
        return LCDHIP_OK;
    hipError_t status = hipModuleUnload(module->module);
    delete module;
    if (status != hipSuccess) {
        set_error("hipModuleUnload: %s", hipGetErrorString(status));
        return LCDHIP_ERR_HIP;
    }
    return LCDHIP_OK;
}

extern "C" int lcdhip_module_get_kernel(lcdhip_module *module, const char *name,
                                        lcdhip_kernel **out)
{
    LCDHIP_REQUIRE_INIT();
    if (!module || !name || !out) {
        set_error("module/name/out must not be NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    hipFunction_t function = nullptr;
    hipError_t status = hipModuleGetFunction(&function, module->module, name);
    if (status != hipSuccess) {
        set_error("generated symbol '%s' was not bound: %s", name,
                  hipGetErrorString(status));
        return LCDHIP_ERR_HIP;
    }
    auto *kernel = new lcdhip_kernel();
    kernel->function = function;
    *out = kernel;  // owned by the module's lifetime; small, freed at unload
    return LCDHIP_OK;
}

extern "C" int lcdhip_kernel_max_resident_blocks(lcdhip_kernel *kernel,
                                                 int block_threads,
                                                 size_t lds_bytes,
                                                 int *blocks_out)
{
    LCDHIP_REQUIRE_INIT();
    if (!kernel || !blocks_out || block_threads <= 0) {
        set_error("bad kernel/blocks_out/block_threads");
        return LCDHIP_ERR_ARGUMENT;
    }
    int per_cu = 0;
    LCDHIP_CHECK(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, kernel->function, block_threads, lds_bytes));
    *blocks_out = per_cu * context().props.multiProcessorCount;
    return LCDHIP_OK;
}

extern "C" int lcdhip_launch(lcdhip_kernel *kernel, uint32_t grid_x,
                             uint32_t block_x, size_t lds_bytes,
                             lcdhip_stream stream, void **args)
{
    LCDHIP_REQUIRE_INIT();
    if (!kernel || block_x == 0 || block_x > 1024) {
        set_error("bad kernel handle or block size %u", block_x);
        return LCDHIP_ERR_ARGUMENT;
    }
    if (grid_x == 0)
        return LCDHIP_OK;
    LCDHIP_CHECK(hipModuleLaunchKernel(kernel->function, grid_x, 1, 1, block_x,
                                       1, 1, static_cast<unsigned>(lds_bytes),
                                       resolve_stream(stream), args, nullptr));
    return LCDHIP_OK;
}

extern "C" int lcdhip_launch_levels(lcdhip_kernel *kernel,
                                    const int32_t *host_ptr,
                                    int64_t level_count, int32_t tasks_per_block,
                                    uint32_t block_x, size_t lds_bytes,
                                    lcdhip_stream stream, void **args,
                                    int start_arg, int end_arg)
{
    LCDHIP_REQUIRE_INIT();
    if (!kernel || !host_ptr || !args || tasks_per_block <= 0 || block_x == 0 ||
        block_x > 1024 || start_arg < 0 || end_arg < 0) {
        set_error("bad argument to lcdhip_launch_levels");
        return LCDHIP_ERR_ARGUMENT;
    }
    hipStream_t hip_stream = resolve_stream(stream);
    for (int64_t level = 0; level < level_count; ++level) {
        int32_t begin = host_ptr[level], end = host_ptr[level + 1];
        if (end <= begin)
            continue;
        *static_cast<int32_t *>(args[start_arg]) = begin;
        *static_cast<int32_t *>(args[end_arg]) = end;
        uint32_t blocks = static_cast<uint32_t>(
            (static_cast<int64_t>(end) - begin + tasks_per_block - 1) /
            tasks_per_block);
        LCDHIP_CHECK(hipModuleLaunchKernel(
            kernel->function, blocks, 1, 1, block_x, 1, 1,
            static_cast<unsigned>(lds_bytes), hip_stream, args, nullptr));
    }
    return LCDHIP_OK;
}

// ------------------------------------------------------------- graphs ----

extern "C" int lcdhip_graph_begin_capture(lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    LCDHIP_CHECK(hipStreamBeginCapture(resolve_stream(stream),
                                       hipStreamCaptureModeRelaxed));
    lcdhip::g_open_captures.fetch_add(1);
    return LCDHIP_OK;
}

extern "C" int lcdhip_graph_end_capture(lcdhip_stream stream, lcdhip_graph **out)
{
    LCDHIP_REQUIRE_INIT();
    auto *graph = new lcdhip_graph();
    hipError_t status = hipStreamEndCapture(resolve_stream(stream), &graph->graph);
    if (lcdhip::g_open_captures.load() > 0)
        lcdhip::g_open_captures.fetch_sub(1);
    if (status != hipSuccess) {
        set_error("hipStreamEndCapture: %s", hipGetErrorString(status));
        delete graph;
        return LCDHIP_ERR_HIP;
    }
    status = hipGraphInstantiate(&graph->exec, graph->graph, nullptr, nullptr, 0);
    if (status != hipSuccess) {
        set_error("hipGraphInstantiate: %s", hipGetErrorString(status));
        (void)hipGraphDestroy(graph->graph);
        delete graph;
        return LCDHIP_ERR_HIP;
    }
    *out = graph;
    return LCDHIP_OK;
}

extern "C" int lcdhip_graph_launch(lcdhip_graph *graph, lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (!graph) {
        set_error("graph is NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    LCDHIP_CHECK(hipGraphLaunch(graph->exec, resolve_stream(stream)));
    return LCDHIP_OK;
}

extern "C" int lcdhip_graph_destroy(lcdhip_graph *graph)
{
    if (!graph)
        return LCDHIP_OK;
    (void)hipGraphExecDestroy(graph->exec);
    (void)hipGraphDestroy(graph->graph);
    delete graph;
    return LCDHIP_OK;
}

// ------------------------------------------------------ lookup tables ----

// One lane per segment.  status[0] collects the worst error seen:
// 1 = pointer array not monotone / out of range, 2 = unsorted segment.
__global__ void lcdhip_lookup_kernel(const int32_t *__restrict__ ptr,
                                     const int32_t *__restrict__ idx, int64_t n,
                                     int64_t idx_size,
                                     int32_t *__restrict__ positions,
                                     int32_t *status)
{
    int64_t s = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (s >= n)
        return;
    int64_t start = ptr[s], end = ptr[s + 1];
    int32_t found = -1;
    if (start < 0 || end < start || end > idx_size) {
        atomicMax(status, 1);
        positions[s] = -1;
        return;
    }
    bool sorted = true;
    for (int64_t p = start + 1; p < end; ++p)
        sorted = sorted && idx[p] >= idx[p - 1];
    if (!sorted)
        atomicMax(status, 2);
    int64_t lo = start, hi = end;
    while (lo < hi) {
        int64_t mid = (lo + hi) >> 1;
        if (idx[mid] < s)
            lo = mid + 1;
        else
            hi = mid;
    }
    if (lo < end && idx[lo] == s)
        found = static_cast<int32_t>(lo);
    positions[s] = found;
}

extern "C" int lcdhip_lookup_build(const int32_t *d_ptr, const int32_t *d_idx,
                                   int64_t n, int64_t idx_size,
                                   int32_t *d_positions, lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (n < 0 || !d_ptr || (n > 0 && !d_positions)) {
        set_error("bad argument to lcdhip_lookup_build");
        return LCDHIP_ERR_ARGUMENT;
    }
    hipStream_t hip_stream = resolve_stream(stream);
    int32_t *d_status = nullptr;
    LCDHIP_CHECK(hipMalloc(&d_status, 4));
    LCDHIP_CHECK(hipMemsetAsync(d_status, 0, 4, hip_stream));
    if (n > 0) {
        unsigned blocks = static_cast<unsigned>((n + 255) / 256);
        hipLaunchKernelGGL(lcdhip_lookup_kernel, dim3(blocks), dim3(256), 0,
                           hip_stream, d_ptr, d_idx, n, idx_size, d_positions,
                           d_status);
    }
    int32_t status = 0;
    hipError_t copy_status = hipMemcpyAsync(&status, d_status, 4,
                                            hipMemcpyDeviceToHost, hip_stream);
    if (copy_status == hipSuccess)
        copy_status = hipStreamSynchronize(hip_stream);
    (void)hipFree(d_status);
    if (copy_status != hipSuccess) {
        set_error("lookup kernel failed: %s", hipGetErrorString(copy_status));
        return LCDHIP_ERR_HIP;
    }
    if (status == 1) {
        set_error("invalid pointer segment in the structural lookup arrays");
        return LCDHIP_ERR_LOOKUP_POINTER;
    }
    if (status == 2) {
        set_error("a segment violates the segmented_monotonically_increasing "
                  "property");
        return LCDHIP_ERR_LOOKUP_ORDER;
    }
    return LCDHIP_OK;
}

// ---- pair table: where segment idx[p] holds the entries of p's own segment
// base[s] = sum over the segments before s of (their length)^2; for the
// segment s with entries a, b in [0, len): table[base[s] + a * len + b] = first
// position in segment idx[ptr[s] + a] whose index equals idx[ptr[s] + b], or -1.

__global__ void lcdhip_pair_square_kernel(const int32_t *__restrict__ ptr,
                                          int64_t n, int64_t idx_size,
                                          int64_t longest,
                                          unsigned long long *__restrict__ total,
                                          int32_t *status)
{
    int64_t s = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    unsigned long long mine = 0;
    if (s < n) {
        const int64_t start = ptr[s], end = ptr[s + 1];
        if (start < 0 || end < start || end > idx_size)
            atomicMax(status, 2);
        else if (end - start > longest)
            atomicMax(status, 1);
        else
            mine = static_cast<unsigned long long>(end - start) * (end - start);
    }
    for (int offset = 32; offset > 0; offset >>= 1)
        mine += __shfl_xor(mine, offset, 64);
    if ((threadIdx.x & 63) == 0 && mine)
        atomicAdd(total, mine);
}

// one workgroup scans the squares; 2^31 entries at most, so 32-bit sums do
__global__ void __launch_bounds__(1024)
lcdhip_pair_base_kernel(const int32_t *__restrict__ ptr, int64_t n,
                        int32_t *__restrict__ base)
{
    __shared__ unsigned int carry, wave_total[16];
    if (threadIdx.x == 0)
        carry = 0;
    __syncthreads();
    for (int64_t first = 0; first < n; first += 1024) {
        const int64_t s = first + threadIdx.x;
        unsigned int len = s < n ? static_cast<unsigned int>(ptr[s + 1] - ptr[s]) : 0u;
        unsigned int value = len * len, scan = value;
        for (int offset = 1; offset < 64; offset <<= 1) {
            const unsigned int up = __shfl_up(scan, offset, 64);
            if ((threadIdx.x & 63) >= offset)
                scan += up;
        }
        if ((threadIdx.x & 63) == 63)
            wave_total[threadIdx.x >> 6] = scan;
        __syncthreads();
        unsigned int before = carry;
        for (unsigned w = 0; w < (threadIdx.x >> 6); ++w)
            before += wave_total[w];
        if (s < n)
            base[s] = static_cast<int32_t>(before + scan - value);
        __syncthreads();
        if (threadIdx.x == 1023)
            carry = before + scan;
        __syncthreads();
    }
    if (threadIdx.x == 0)
        base[n] = static_cast<int32_t>(carry);
}

// T = int32_t: positions in idx; T = int8_t: offsets from the start of the
// segment searched (segments of at most 127 entries)
template <class T>
__global__ void lcdhip_pair_fill_kernel(const int32_t *__restrict__ ptr,
                                        const int32_t *__restrict__ idx,
                                        int64_t n, int64_t idx_size,
                                        const int32_t *__restrict__ base,
                                        T *__restrict__ table)
{
    int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p >= idx_size || p < ptr[0] || p >= ptr[n])
        return;
    // the segment that holds position p
    int64_t lo = 0, hi = n;
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (ptr[mid] <= p)
            lo = mid;
        else
            hi = mid;
    }
    const int64_t s = lo, start = ptr[s], len = ptr[s + 1] - start;
    const int64_t k = idx[p];
    T *row = table + base[s] + (p - start) * len;
    const bool valid = k >= 0 && k < n;
    const int64_t k_start = valid ? ptr[k] : 0, k_end = valid ? ptr[k + 1] : 0;
    for (int64_t b = 0; b < len; ++b) {
        const int32_t key = idx[start + b];
        int64_t left = k_start, right = k_end;
        while (left < right) {
            const int64_t mid = (left + right) >> 1;
            if (idx[mid] < key)
                left = mid + 1;
            else
                right = mid;
        }
        const bool found = left < k_end && idx[left] == key;
        row[b] = static_cast<T>(!found ? -1 : sizeof(T) == 1 ? left - k_start : left);
    }
}

static int pair_table_build(const int32_t *d_ptr, const int32_t *d_idx, int64_t n,
                            int64_t idx_size, int32_t *d_base, void *d_table,
                            int element_bytes, int64_t capacity,
                            int64_t *entries_out, lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (n < 0 || idx_size < 0 || capacity < 0 || !d_ptr || !entries_out ||
        (idx_size > 0 && !d_idx) || (d_table && !d_base)) {
        set_error("bad argument to the pair table build");
        return LCDHIP_ERR_ARGUMENT;
    }
    const int64_t longest = element_bytes == 1 ? 127 : INT64_MAX;
    hipStream_t hip_stream = resolve_stream(stream);
    *entries_out = 0;
    unsigned long long *d_total = nullptr;
    LCDHIP_CHECK(hipMalloc(&d_total, 16));
    int32_t *d_status = reinterpret_cast<int32_t *>(d_total + 1);
    hipError_t error = hipMemsetAsync(d_total, 0, 16, hip_stream);
    unsigned long long host[2] = {0, 0};
    if (error == hipSuccess && n > 0)
        hipLaunchKernelGGL(lcdhip_pair_square_kernel,
                           dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                           0, hip_stream, d_ptr, n, idx_size, longest, d_total,
                           d_status);
    if (error == hipSuccess)
        error = hipMemcpyAsync(host, d_total, 16, hipMemcpyDeviceToHost, hip_stream);
    if (error == hipSuccess)
        error = hipStreamSynchronize(hip_stream);
    (void)hipFree(d_total);
    if (error != hipSuccess) {
        set_error("pair table sizing failed: %s", hipGetErrorString(error));
        return LCDHIP_ERR_HIP;
    }
    if (static_cast<int32_t>(host[1] & 0xffffffffu) == 2) {
        set_error("invalid pointer segment in the structural lookup arrays");
        return LCDHIP_ERR_LOOKUP_POINTER;
    }
    if (static_cast<int32_t>(host[1] & 0xffffffffu) == 1) {
        set_error("a segment of more than 127 entries: its offsets do not fit a byte");
        return LCDHIP_ERR_ARGUMENT;
    }
    if (host[0] >= (1ull << 31)) {
        set_error("a pair table of %llu entries exceeds 2^31", host[0]);
        return LCDHIP_ERR_ARGUMENT;
    }
    *entries_out = static_cast<int64_t>(host[0]);
    if (!d_table)
        return LCDHIP_OK;
    if (capacity < *entries_out) {
        set_error("pair table buffer too small: %lld < %lld",
                  static_cast<long long>(capacity),
                  static_cast<long long>(*entries_out));
        return LCDHIP_ERR_ARGUMENT;
    }
    hipLaunchKernelGGL(lcdhip_pair_base_kernel, dim3(1), dim3(1024), 0, hip_stream,
                       d_ptr, n, d_base);
    if (idx_size > 0 && n > 0 && element_bytes == 1)
        hipLaunchKernelGGL(lcdhip_pair_fill_kernel<int8_t>,
                           dim3(static_cast<unsigned>((idx_size + 255) / 256)),
                           dim3(256), 0, hip_stream, d_ptr, d_idx, n, idx_size,
                           d_base, static_cast<int8_t *>(d_table));
    else if (idx_size > 0 && n > 0)
        hipLaunchKernelGGL(lcdhip_pair_fill_kernel<int32_t>,
                           dim3(static_cast<unsigned>((idx_size + 255) / 256)),
                           dim3(256), 0, hip_stream, d_ptr, d_idx, n, idx_size,
                           d_base, static_cast<int32_t *>(d_table));
    LCDHIP_CHECK(hipGetLastError());
    LCDHIP_CHECK(hipStreamSynchronize(hip_stream));
    return LCDHIP_OK;
}

extern "C" int lcdhip_pair_lookup_build(const int32_t *d_ptr, const int32_t *d_idx,
                                        int64_t n, int64_t idx_size,
                                        int32_t *d_base, int32_t *d_table,
                                        int64_t capacity, int64_t *entries_out,
                                        lcdhip_stream stream)
{
    return pair_table_build(d_ptr, d_idx, n, idx_size, d_base, d_table, 4,
                            capacity, entries_out, stream);
}

extern "C" int lcdhip_pair_offsets_build(const int32_t *d_ptr, const int32_t *d_idx,
                                         int64_t n, int64_t idx_size,
                                         int32_t *d_base, int8_t *d_table,
                                         int64_t capacity, int64_t *entries_out,
                                         lcdhip_stream stream)
{
    return pair_table_build(d_ptr, d_idx, n, idx_size, d_base, d_table, 1,
                            capacity, entries_out, stream);
}

// -------------------------------------------------------------- digest ----

__device__ inline uint64_t lcdhip_mix64(uint64_t x)
{
    x ^= x >> 30;
    x *= 0xbf58476d1ce4e5b9ull;
    x ^= x >> 27;
    x *= 0x94d049bb133111ebull;
    x ^= x >> 31;
    return x;
}

// Position-salted word hashes combined with + and ^ (both commutative and
// associative, so the digest does not depend on how the words are dealt out to
// lanes and workgroups).  Every workgroup leaves one pair of partial results
// in partial[2 * blockIdx.x ..]; no atomics, nothing to clear beforehand.
#define LCDHIP_DIGEST_MAX_BLOCKS 1024
#define LCDHIP_DIGEST_THREADS 256

__global__ void __launch_bounds__(LCDHIP_DIGEST_THREADS)
lcdhip_digest_partial_kernel(const uint32_t *__restrict__ words, size_t count,
                             unsigned long long *__restrict__ partial)
{
    __shared__ unsigned long long wave_sum[LCDHIP_DIGEST_THREADS / 64];
    __shared__ unsigned long long wave_mix[LCDHIP_DIGEST_THREADS / 64];
    size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    uint64_t sum = 0, mixed = 0;
    for (; i < count; i += stride) {
        uint64_t h = lcdhip_mix64((static_cast<uint64_t>(words[i]) << 32) ^
                                  (i * 0x9e3779b97f4a7c15ull + 1));
        sum += h;
        mixed ^= lcdhip_mix64(h + 0x632be59bd9b4e019ull);
    }
    for (int offset = 32; offset > 0; offset >>= 1) {
        sum += __shfl_down(sum, offset);
        mixed ^= __shfl_down(mixed, offset);
    }
    if ((threadIdx.x & 63) == 0) {
        wave_sum[threadIdx.x >> 6] = sum;
        wave_mix[threadIdx.x >> 6] = mixed;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < LCDHIP_DIGEST_THREADS / 64; ++w) {
            sum += wave_sum[w];
            mixed ^= wave_mix[w];
        }
        partial[2 * blockIdx.x] = sum;
        partial[2 * blockIdx.x + 1] = mixed;
    }
}

// One workgroup folds the first `blocks` pairs (whatever lies behind them is
// ignored) and salts the sum with the length.
__global__ void __launch_bounds__(LCDHIP_DIGEST_THREADS)
lcdhip_digest_final_kernel(const unsigned long long *__restrict__ partial,
                           int blocks, unsigned long long bytes,
                           unsigned long long *__restrict__ out)
{
    __shared__ unsigned long long wave_sum[LCDHIP_DIGEST_THREADS / 64];
    __shared__ unsigned long long wave_mix[LCDHIP_DIGEST_THREADS / 64];
    uint64_t sum = 0, mixed = 0;
    for (int b = threadIdx.x; b < blocks; b += LCDHIP_DIGEST_THREADS) {
        sum += partial[2 * b];
        mixed ^= partial[2 * b + 1];
    }
    for (int offset = 32; offset > 0; offset >>= 1) {
        sum += __shfl_down(sum, offset);
        mixed ^= __shfl_down(mixed, offset);
    }
    if ((threadIdx.x & 63) == 0) {
        wave_sum[threadIdx.x >> 6] = sum;
        wave_mix[threadIdx.x >> 6] = mixed;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < LCDHIP_DIGEST_THREADS / 64; ++w) {
            sum += wave_sum[w];
            mixed ^= wave_mix[w];
        }
        out[0] = sum ^ (bytes * 0x9e3779b97f4a7c15ull);
        out[1] = mixed;
    }
}

// Both digest entry points: partial results into `d_partial` (room for
// 2 * LCDHIP_DIGEST_MAX_BLOCKS words), the digest into d_out[0..1].
static int digest_enqueue(const void *d_data, size_t bytes,
                          unsigned long long *d_partial,
                          unsigned long long *d_out, hipStream_t hip_stream)
{
    size_t count = bytes / 4;
    int blocks = static_cast<int>(std::min<size_t>(
        (count + LCDHIP_DIGEST_THREADS - 1) / LCDHIP_DIGEST_THREADS,
        LCDHIP_DIGEST_MAX_BLOCKS));
    if (blocks) {
        hipLaunchKernelGGL(lcdhip_digest_partial_kernel, dim3(blocks),
                           dim3(LCDHIP_DIGEST_THREADS), 0, hip_stream,
                           static_cast<const uint32_t *>(d_data), count,
                           d_partial);
        LCDHIP_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(lcdhip_digest_final_kernel, dim3(1),
                       dim3(LCDHIP_DIGEST_THREADS), 0, hip_stream, d_partial,
                       blocks, static_cast<unsigned long long>(bytes), d_out);
    LCDHIP_CHECK(hipGetLastError());
    return LCDHIP_OK;
}

extern "C" int lcdhip_digest(const void *d_data, size_t bytes, uint64_t out[2],
                             lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (!out || (bytes & 3) || (bytes && !d_data)) {
        set_error("digest needs data, out and a multiple of 4 bytes");
        return LCDHIP_ERR_ARGUMENT;
    }
    hipStream_t hip_stream = resolve_stream(stream);
    unsigned long long *d_work = nullptr;   // partial results, then the digest
    const size_t partial_words = 2 * LCDHIP_DIGEST_MAX_BLOCKS;
    LCDHIP_CHECK(hipMalloc(&d_work, (partial_words + 2) * 8));
    int enqueued = digest_enqueue(d_data, bytes, d_work, d_work + partial_words,
                                  hip_stream);
    hipError_t status = hipSuccess;
    if (enqueued == LCDHIP_OK) {
        status = hipMemcpyAsync(out, d_work + partial_words, 16,
                                hipMemcpyDeviceToHost, hip_stream);
        if (status == hipSuccess)
            status = hipStreamSynchronize(hip_stream);
    }
    (void)hipFree(d_work);
    if (enqueued != LCDHIP_OK)
        return enqueued;
    if (status != hipSuccess) {
        set_error("digest failed: %s", hipGetErrorString(status));
        return LCDHIP_ERR_HIP;
    }
    return LCDHIP_OK;
}

extern "C" int lcdhip_digest_noalloc(const void *d_data, size_t bytes,
                                     uint64_t *d_out, lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    static_assert(LCDHIP_DIGEST_SCRATCH_WORDS >= 2 * LCDHIP_DIGEST_MAX_BLOCKS,
                  "scratch must hold one pair per workgroup");
    if (!d_out || (bytes & 3) || (bytes && !d_data)) {
        set_error("lcdhip_digest_noalloc needs data, d_out and a multiple of "
                  "4 bytes");
        return LCDHIP_ERR_ARGUMENT;
    }
    if (bytes > LCDHIP_DIGEST_NOALLOC_MAX_BYTES) {
        set_error("lcdhip_digest_noalloc: %zu bytes exceed the limit of %zu",
                  bytes, static_cast<size_t>(LCDHIP_DIGEST_NOALLOC_MAX_BYTES));
        return LCDHIP_ERR_ARGUMENT;
    }
    const int device = context().device;
    unsigned long long *scratch =
        device >= 0 && device < LCDHIP_MAX_DEVICES ? g_digest_scratch[device]
                                                   : nullptr;
    if (!scratch) {
        set_error("lcdhip_digest_noalloc: no work area on device %d", device);
        return LCDHIP_ERR_ARGUMENT;
    }
    return digest_enqueue(d_data, bytes, scratch,
                          reinterpret_cast<unsigned long long *>(d_out),
                          resolve_stream(stream));
}

// ---------------------------------------------------- machine constants ----

__global__ void lcdhip_empty_kernel() {}

// What one level of a level-synchronous executor at least does: a chain of
// three dependent loads (task -> segment bounds -> operand) and a store.
__global__ void lcdhip_level_probe_kernel(const int32_t *__restrict__ chain,
                                          int32_t *out, int32_t mask)
{
    int32_t v = static_cast<int32_t>(threadIdx.x + blockIdx.x);
    v = chain[v & mask];
    v = chain[v & mask];
    v = chain[v & mask];
    out[threadIdx.x] = v;
}

__global__ void lcdhip_release_probe_kernel(int32_t *counters, int32_t nodes,
                                            int32_t stride)
{
    if (threadIdx.x == 0) {
        int32_t node = blockIdx.x;
        atomicSub(&counters[(static_cast<int64_t>(node) * stride) % nodes], 1);
    }
}

__global__ void lcdhip_copy_probe_kernel(const float4 *__restrict__ src,
                                         float4 *__restrict__ dst, size_t count)
{
    size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (; i < count; i += stride)
        dst[i] = src[i];
}

// Two workgroups bounce a flag `hops` times.  Consecutive workgroup ids land
// on different XCDs, so the hop crosses L2s: the cost a dependent task pays in
// the sync-free executor.  Every wait is bounded.
__global__ void lcdhip_handoff_probe_kernel(int32_t *flag, int32_t hops,
                                            int32_t *timed_out)
{
    if (threadIdx.x != 0 || blockIdx.x > 1)
        return;
    const int32_t me = blockIdx.x;
    for (int32_t hop = me; hop < hops; hop += 2) {
        int64_t spins = 0;
        while (__hip_atomic_load(flag, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) != hop) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > (1ll << 22)) {
                *timed_out = 1;
                return;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_store(flag, hop + 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Two wavefronts of ONE workgroup hand a word back and forth through LDS: the
// hop a dependent task pays when its producer runs in the same workgroup
// (tiles, faces between the bundles of a grid sweep).  Every wait is bounded.
__global__ void lcdhip_lds_handoff_probe_kernel(int32_t hops, int32_t *timed_out)
{
    __shared__ int32_t flag;
    if (threadIdx.x == 0)
        flag = 0;
    __syncthreads();
    const int32_t me = static_cast<int32_t>(threadIdx.x >> 6);
    if ((threadIdx.x & 63) != 0 || me > 1)
        return;
    for (int32_t hop = me; hop < hops; hop += 2) {
        int64_t spins = 0;
        while (__hip_atomic_load(&flag, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP) != hop) {
            if (++spins > (1ll << 22)) {
                *timed_out = 1;
                return;
            }
        }
        __hip_atomic_store(&flag, hop + 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

// One wavefront runs `steps` dependent steps x = (b - c * x) / d in fp64: what
// a chain of tasks of a triangular solve costs when every hand-off is free (a
// register of the same lane): no executor of such a chain can be faster.
__global__ void lcdhip_chain_probe_kernel(double *out, int32_t steps, double b,
                                          double c, double d)
{
    double x = out[threadIdx.x];
    for (int32_t step = 0; step < steps; ++step)
        x = (b - c * x) / d;
    out[threadIdx.x] = x;
}

// `rounds` barriers over a grid that the host sized to be fully resident.
__global__ void lcdhip_barrier_probe_kernel(int32_t *arrive, int32_t rounds,
                                            int32_t *timed_out)
{
    for (int32_t round = 0; round < rounds; ++round) {
        __syncthreads();
        if (threadIdx.x == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __hip_atomic_fetch_add(&arrive[round], 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            int64_t spins = 0;
            while (__hip_atomic_load(&arrive[round], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) <
                   static_cast<int32_t>(gridDim.x)) {
                __builtin_amdgcn_s_sleep(1);
                if (++spins > (1ll << 22)) {
                    *timed_out = 1;
                    break;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        __syncthreads();
    }
}

static double median(std::vector<double> samples)
{
    std::sort(samples.begin(), samples.end());
    return samples[samples.size() / 2];
}

extern "C" int lcdhip_measure_arch(lcdhip_arch *out)
{
    LCDHIP_REQUIRE_INIT();
    if (!out) {
        set_error("out is NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    auto &ctx = context();
    hipStream_t stream = ctx.stream;
    memset(out, 0, sizeof(*out));
    using clock = std::chrono::steady_clock;

    // launch + synchronise round trip (compiler/scheduler.py:741-754)
    hipLaunchKernelGGL(lcdhip_empty_kernel, dim3(1), dim3(1), 0, stream);
    LCDHIP_CHECK(hipStreamSynchronize(stream));
    std::vector<double> samples;
    for (int repeat = 0; repeat < 64; ++repeat) {
        auto start = clock::now();
        hipLaunchKernelGGL(lcdhip_empty_kernel, dim3(1), dim3(1), 0, stream);
        LCDHIP_CHECK(hipStreamSynchronize(stream));
        samples.push_back(
            std::chrono::duration<double>(clock::now() - start).count());
    }
    out->launch_latency_s = median(samples);

    hipEvent_t start_event, stop_event;
    LCDHIP_CHECK(hipEventCreate(&start_event));
    LCDHIP_CHECK(hipEventCreate(&stop_event));
    float ms = 0.f;

    // release cost per node (compiler/scheduler.py:757-775)
    const int32_t nodes = 1 << 16;
    int32_t *d_counters = nullptr;
    LCDHIP_CHECK(hipMalloc(&d_counters, nodes * 4));
    LCDHIP_CHECK(hipMemsetAsync(d_counters, 0, nodes * 4, stream));
    hipLaunchKernelGGL(lcdhip_release_probe_kernel, dim3(nodes), dim3(64), 0,
                       stream, d_counters, nodes, 7919);
    samples.clear();
    for (int repeat = 0; repeat < 5; ++repeat) {
        LCDHIP_CHECK(hipEventRecord(start_event, stream));
        hipLaunchKernelGGL(lcdhip_release_probe_kernel, dim3(nodes), dim3(64),
                           0, stream, d_counters, nodes, 7919);
        LCDHIP_CHECK(hipEventRecord(stop_event, stream));
        LCDHIP_CHECK(hipEventSynchronize(stop_event));
        LCDHIP_CHECK(hipEventElapsedTime(&ms, start_event, stop_event));
        samples.push_back(ms * 1.0e-3 / nodes);
    }
    out->atomic_cost_s = median(samples);
    LCDHIP_CHECK(hipFree(d_counters));

    // streaming copy bandwidth (read + write bytes)
    const size_t copy_bytes = size_t(1) << 30;
    float4 *d_src = nullptr, *d_dst = nullptr;
    LCDHIP_CHECK(hipMalloc(&d_src, copy_bytes));
    LCDHIP_CHECK(hipMalloc(&d_dst, copy_bytes));
    LCDHIP_CHECK(hipMemsetAsync(d_src, 1, copy_bytes, stream));
    samples.clear();
    for (int repeat = 0; repeat < 6; ++repeat) {
        LCDHIP_CHECK(hipEventRecord(start_event, stream));
        hipLaunchKernelGGL(lcdhip_copy_probe_kernel, dim3(8192), dim3(256), 0,
                           stream, d_src, d_dst, copy_bytes / 16);
        LCDHIP_CHECK(hipEventRecord(stop_event, stream));
        LCDHIP_CHECK(hipEventSynchronize(stop_event));
        LCDHIP_CHECK(hipEventElapsedTime(&ms, start_event, stop_event));
        if (repeat)
            samples.push_back(2.0 * copy_bytes / (ms * 1.0e-3));
    }
    out->memory_bandwidth_bytes_per_s = median(samples);
    LCDHIP_CHECK(hipFree(d_src));
    LCDHIP_CHECK(hipFree(d_dst));

    out->lane_flops_per_s = ctx.props.clockRate * 1.0e3;

    // cross-workgroup hand-off
    int32_t *d_flags = nullptr;
    const int32_t rounds = 256;
    LCDHIP_CHECK(hipMalloc(&d_flags, (rounds + 8) * 4));
    int32_t *d_timed_out = d_flags + rounds + 4;
    const int32_t hops = 2000;
    samples.clear();
    for (int repeat = 0; repeat < 4; ++repeat) {
        LCDHIP_CHECK(hipMemsetAsync(d_flags, 0, (rounds + 8) * 4, stream));
        LCDHIP_CHECK(hipEventRecord(start_event, stream));
        hipLaunchKernelGGL(lcdhip_handoff_probe_kernel, dim3(2), dim3(64), 0,
                           stream, d_flags, hops, d_timed_out);
        LCDHIP_CHECK(hipEventRecord(stop_event, stream));
        LCDHIP_CHECK(hipEventSynchronize(stop_event));
        LCDHIP_CHECK(hipEventElapsedTime(&ms, start_event, stop_event));
        if (repeat)
            samples.push_back(ms * 1.0e-3 / hops);
    }
    out->handoff_s = median(samples);

    // the same ping-pong between two wavefronts of one workgroup, through LDS
    samples.clear();
    for (int repeat = 0; repeat < 4; ++repeat) {
        LCDHIP_CHECK(hipEventRecord(start_event, stream));
        hipLaunchKernelGGL(lcdhip_lds_handoff_probe_kernel, dim3(1), dim3(128),
                           0, stream, hops, d_timed_out);
        LCDHIP_CHECK(hipEventRecord(stop_event, stream));
        LCDHIP_CHECK(hipEventSynchronize(stop_event));
        LCDHIP_CHECK(hipEventElapsedTime(&ms, start_event, stop_event));
        if (repeat)
            samples.push_back(ms * 1.0e-3 / hops);
    }
    out->lds_handoff_s = median(samples);

    // a chain of dependent fp64 steps (multiply, subtract, divide) in one lane;
    // the launch itself is taken out with a second, shorter run
    samples.clear();
    {
        double *d_chain = reinterpret_cast<double *>(d_flags);
        const int32_t long_steps = 20000, short_steps = 2000;
        float ms_long = 0.0f, ms_short = 0.0f;
        for (int repeat = 0; repeat < 4; ++repeat) {
            LCDHIP_CHECK(hipMemsetAsync(d_flags, 0, 64 * 8, stream));
            LCDHIP_CHECK(hipEventRecord(start_event, stream));
            hipLaunchKernelGGL(lcdhip_chain_probe_kernel, dim3(1), dim3(64), 0,
                               stream, d_chain, long_steps, 1.0, -0.25, 6.0);
            LCDHIP_CHECK(hipEventRecord(stop_event, stream));
            LCDHIP_CHECK(hipEventSynchronize(stop_event));
            LCDHIP_CHECK(hipEventElapsedTime(&ms_long, start_event, stop_event));
            LCDHIP_CHECK(hipEventRecord(start_event, stream));
            hipLaunchKernelGGL(lcdhip_chain_probe_kernel, dim3(1), dim3(64), 0,
                               stream, d_chain, short_steps, 1.0, -0.25, 6.0);
            LCDHIP_CHECK(hipEventRecord(stop_event, stream));
            LCDHIP_CHECK(hipEventSynchronize(stop_event));
            LCDHIP_CHECK(hipEventElapsedTime(&ms_short, start_event, stop_event));
            if (repeat && ms_long > ms_short)
                samples.push_back((ms_long - ms_short) * 1.0e-3 /
                                  (long_steps - short_steps));
        }
    }
    out->chain_step_s = samples.empty() ? 0.0 : median(samples);

    // grid barrier over one workgroup per CU
    samples.clear();
    const int barrier_blocks = ctx.props.multiProcessorCount;
    for (int repeat = 0; repeat < 4; ++repeat) {
        LCDHIP_CHECK(hipMemsetAsync(d_flags, 0, (rounds + 8) * 4, stream));
        LCDHIP_CHECK(hipEventRecord(start_event, stream));
        hipLaunchKernelGGL(lcdhip_barrier_probe_kernel, dim3(barrier_blocks),
                           dim3(256), 0, stream, d_flags, rounds, d_timed_out);
        LCDHIP_CHECK(hipEventRecord(stop_event, stream));
        LCDHIP_CHECK(hipEventSynchronize(stop_event));
        LCDHIP_CHECK(hipEventElapsedTime(&ms, start_event, stop_event));
        if (repeat)
            samples.push_back(ms * 1.0e-3 / rounds);
    }
    out->barrier_s = median(samples);
    int32_t timed_out = 0;
    LCDHIP_CHECK(hipMemcpy(&timed_out, d_timed_out, 4, hipMemcpyDeviceToHost));
    LCDHIP_CHECK(hipFree(d_flags));
    if (timed_out) {
        set_error("a machine-constant probe gave up waiting");
        return LCDHIP_ERR_WATCHDOG;
    }

    // per-node cost of a captured chain of dependent launches, each doing
    // the minimal work of one level (three dependent loads and a store)
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    const int chain = 256;
    const int32_t probe_words = 1 << 16;
    int32_t *d_probe = nullptr;
    {
        std::vector<int32_t> host_probe(probe_words + 64);
        for (int32_t w = 0; w < probe_words; ++w)
            host_probe[w] = static_cast<int32_t>(
                (static_cast<int64_t>(w) * 40503 + 12345) & (probe_words - 1));
        LCDHIP_CHECK(hipMalloc(&d_probe, host_probe.size() * 4));
        LCDHIP_CHECK(hipMemcpy(d_probe, host_probe.data(),
                               host_probe.size() * 4, hipMemcpyHostToDevice));
    }
    LCDHIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
    for (int node = 0; node < chain; ++node)
        hipLaunchKernelGGL(lcdhip_level_probe_kernel, dim3(1 + node % 7),
                           dim3(64), 0, stream, d_probe, d_probe + probe_words,
                           probe_words - 1);
    LCDHIP_CHECK(hipStreamEndCapture(stream, &graph));
    LCDHIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    samples.clear();
    for (int repeat = 0; repeat < 5; ++repeat) {
        LCDHIP_CHECK(hipEventRecord(start_event, stream));
        LCDHIP_CHECK(hipGraphLaunch(exec, stream));
        LCDHIP_CHECK(hipEventRecord(stop_event, stream));
        LCDHIP_CHECK(hipEventSynchronize(stop_event));
        LCDHIP_CHECK(hipEventElapsedTime(&ms, start_event, stop_event));
        if (repeat)
            samples.push_back(ms * 1.0e-3 / chain);
    }
    out->graph_node_s = median(samples);
    (void)hipFree(d_probe);
    (void)hipGraphExecDestroy(exec);
    (void)hipGraphDestroy(graph);
    (void)hipEventDestroy(start_event);
    (void)hipEventDestroy(stop_event);
    return LCDHIP_OK;
}

__global__ void lcdhip_gather_kernel(int32_t *__restrict__ dst,
                                     const int32_t *__restrict__ src,
                                     const int32_t *__restrict__ index,
                                     int64_t offset, int64_t count,
                                     int64_t src_size, int32_t *status)
{
    int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (q >= count)
        return;
    const int64_t at = static_cast<int64_t>(index[q]) + offset;
    if (at < 0 || at >= src_size) {
        atomicMax(status, 1);
        dst[q] = 0;
        return;
    }
    dst[q] = src[at];
}

extern "C" int lcdhip_gather_i32(int32_t *d_dst, const int32_t *d_src,
                                 const int32_t *d_index, int64_t offset,
                                 int64_t count, int64_t src_size,
                                 lcdhip_stream stream)
{
    LCDHIP_REQUIRE_INIT();
    if (count < 0 || src_size < 0 ||
        (count > 0 && (!d_dst || !d_src || !d_index))) {
        set_error("bad argument to lcdhip_gather_i32");
        return LCDHIP_ERR_ARGUMENT;
    }
    if (count == 0)
        return LCDHIP_OK;
    hipStream_t hip_stream = resolve_stream(stream);
    int32_t *d_status = nullptr;
    LCDHIP_CHECK(hipMalloc(&d_status, 4));
    LCDHIP_CHECK(hipMemsetAsync(d_status, 0, 4, hip_stream));
    hipLaunchKernelGGL(lcdhip_gather_kernel,
                       dim3(static_cast<unsigned>((count + 255) / 256)),
                       dim3(256), 0, hip_stream, d_dst, d_src, d_index, offset,
                       count, src_size, d_status);
    int32_t status = 0;
    hipError_t copy_status = hipMemcpyAsync(&status, d_status, 4,
                                            hipMemcpyDeviceToHost, hip_stream);
    if (copy_status == hipSuccess)
        copy_status = hipStreamSynchronize(hip_stream);
    (void)hipFree(d_status);
    if (copy_status != hipSuccess) {
        set_error("gather kernel failed: %s", hipGetErrorString(copy_status));
        return LCDHIP_ERR_HIP;
    }
    if (status) {
        set_error("lcdhip_gather_i32: an index plus offset leaves the source "
                  "array");
        return LCDHIP_ERR_ARGUMENT;
    }
    return LCDHIP_OK;
}
