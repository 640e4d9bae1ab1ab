// The C ABI of libtensomite_hip.so (include/tensomite_hip.h): devices,
// memory, the buffer layer, errors, events, and the kernel entry points.
//
// Per device the library keeps one ordered stream, a pool of freed device
// memory keyed by exact size with a finalizer-safe retired list in front of
// it, a pinned staging ring for asynchronous uploads, growable scratch for
// quantised activations, and the 12-byte error buffer gather kernels report
// into. This is the host side of the reference's `CUDA < HostDevice`
// (src/tensomite/cuda.cr) and its `BufferPool`/`RetiredList`
// (src/tensomite/buffer_pool.cr), restated natively for HIP.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/tensomite_hip.h"
#include "tmh_internal.h"
#include "tmh_pool.h"

namespace {
std::atomic<int> g_fail_allocations{0};
}  // namespace

namespace tmh {

hipError_t device_malloc(void** p, size_t bytes) {
    int left = g_fail_allocations.load();
    while (left > 0) {
        if (g_fail_allocations.compare_exchange_weak(left, left - 1)) return hipErrorOutOfMemory;
    }
    return hipMalloc(p, bytes);
}

size_t scratch_need(uint32_t rows, uint32_t k) {
    const size_t nb = k / 32u;
    const size_t per = ((size_t)rows * nb * 4u + 255u) & ~(size_t)255u;
    return 3 * per + (((size_t)rows * k + 255u) & ~(size_t)255u);
}

// The quantise pass's four outputs for `rows` rows of k, carved from `base`.
hipError_t make_stream(uint32_t kind, std::vector<StreamProduct>& products, int compute_units, StreamLaunch& l,
                       void** mem, uint32_t wgs_per_cu) {
    *mem = nullptr;
    std::vector<StreamStart> starts;
    if (!plan_stream(kind, products, compute_units, l, starts, wgs_per_cu)) return hipErrorInvalidValue;
    const size_t table_bytes = (sizeof(StreamProduct) * products.size() + 255u) & ~(size_t)255u;
    hipError_t e = device_malloc(mem, table_bytes + sizeof(StreamStart) * starts.size());
    if (e == hipSuccess)
        e = hipMemcpy(*mem, products.data(), sizeof(StreamProduct) * products.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy((uint8_t*)*mem + table_bytes, starts.data(), sizeof(StreamStart) * starts.size(),
                      hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (*mem) (void)hipFree(*mem);
        *mem = nullptr;
        return e;
    }
    l.table = (const StreamProduct*)*mem;
    l.starts = (const StreamStart*)((uint8_t*)*mem + table_bytes);
    return hipSuccess;
}

Activations carve_scratch(uint8_t* base, uint32_t rows, uint32_t k) {
    const size_t nb = k / 32u;
    const size_t per = ((size_t)rows * nb * 4u + 255u) & ~(size_t)255u;
    return Activations{(const float*)base, (const float*)(base + per), (const int32_t*)(base + 2 * per),
                       (const int8_t*)(base + 3 * per)};
}

}  // namespace tmh

// Quantised activations of tmh_block_matmul_fixed: device memory that exists
// from module load to process end, one copy per GPU, so that entry point
// never allocates. Host code must not pass this name to a kernel (on the host
// it is a stand-in, not a device address): each device's address comes from
// hipGetSymbolAddress at set-up (Device::fixed_scratch).
static __device__ __align__(256) uint8_t scratch[TMH_FIXED_SCRATCH_BYTES];

namespace {

using tmh::device_malloc;
using tmh::Pool;
using tmh::Retired;
using tmh::scratch_need;

constexpr int MAX_DEVICES = 16;

// Pinned host memory for asynchronous uploads: SLOTS buffers of SLOT_BYTES,
// used round robin; a slot is reused once the copy out of it has finished.
struct Staging {
    static constexpr int SLOTS = 4;
    static constexpr size_t SLOT_BYTES = 16u << 20;
    void* slot[SLOTS] = {};
    hipEvent_t done[SLOTS] = {};
    bool used[SLOTS] = {};
    int next = 0;
    bool ready = false;
};

struct Device {
    std::mutex setup;
    // Set (release) once the fields below are; read (acquire) before use by
    // any thread.
    std::atomic<bool> ready{false};
    int index = 0;
    hipStream_t stream = nullptr;
    int compute_units = 256;
    uint64_t memory = 0;

    // The error buffer (count, first id, rows), cuda.cr:961-964.
    int32_t* errors = nullptr;
    std::atomic<bool> errors_pending{false};
    int32_t report[3] = {0, 0, 0};
    std::mutex report_lock;  // report is written by tmh_sync, read by tmh_error_report, on any threads

    // Scratch for quantised activations, kept and grown across launches
    // (cuda.cr:788-798); `launch` keeps a quantise pass and its product
    // together.
    std::mutex launch;
    uint8_t* act_scratch = nullptr;
    size_t act_scratch_bytes = 0;

    // This device's copy of the file-scope `scratch` array, looked up once at
    // set-up (the allocation-free entry point's quantised activations), and
    // the lock that keeps its quantise pass and product adjacent on the stream.
    uint8_t* fixed_scratch = nullptr;
    std::mutex fixed_launch;

    Pool pool;
    Retired* retired = nullptr;
    std::mutex staging_lock;
    Staging staging;

    std::atomic<int64_t> uploads{0}, downloads{0}, gpu_ops{0}, device_bytes{0}, frees{0}, launches{0};
};

Device g_devices[MAX_DEVICES];
std::atomic<int> g_count{-1};
std::atomic<bool> g_kernels_off{false};
thread_local int t_device = 0;

int code(hipError_t e) { return (int)e; }

}  // namespace

void tmh::count_launch() {
    const int i = t_device;
    if (i >= 0 && i < MAX_DEVICES) g_devices[i].launches.fetch_add(1, std::memory_order_relaxed);
}

namespace {

int count_devices() {
    int n = g_count.load();
    if (n >= 0) return n;
    int c = 0;
    if (hipGetDeviceCount(&c) != hipSuccess) c = 0;
    if (c > MAX_DEVICES) c = MAX_DEVICES;
    g_count.store(c);
    return c;
}

// Returns the calling thread's device, made current and set up on first
// use, or null with *err set.
Device* current(int* err) {
    const int n = count_devices();
    if (n == 0 || t_device < 0 || t_device >= n) {
        *err = TMH_ERROR_NO_DEVICE;
        return nullptr;
    }
    int now = -1;
    if (hipGetDevice(&now) != hipSuccess || now != t_device) {
        hipError_t e = hipSetDevice(t_device);
        if (e != hipSuccess) {
            *err = code(e);
            return nullptr;
        }
    }
    Device& d = g_devices[t_device];
    if (!d.ready) {
        std::lock_guard<std::mutex> guard(d.setup);
        if (!d.ready) {
            d.index = t_device;
            hipDeviceProp_t prop;
            hipError_t e = hipGetDeviceProperties(&prop, t_device);
            if (e == hipSuccess) {
                d.compute_units = prop.multiProcessorCount;
                d.memory = prop.totalGlobalMem;
                int64_t quarter = (int64_t)(prop.totalGlobalMem / 4);
                d.pool.limit = quarter > (1ll << 30) ? quarter : (1ll << 30);
                e = hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking);
            }
            if (e == hipSuccess) e = hipMalloc((void**)&d.errors, 3 * sizeof(int32_t));
            if (e == hipSuccess) e = hipMemset(d.errors, 0, 3 * sizeof(int32_t));
            if (e == hipSuccess) e = hipGetSymbolAddress((void**)&d.fixed_scratch, HIP_SYMBOL(scratch));
            if (e != hipSuccess) {
                *err = code(e);
                return nullptr;
            }
            d.retired = new Retired();
            d.ready = true;
        }
    }
    *err = TMH_SUCCESS;
    return &d;
}

void recycle_retired(Device& d) {
    d.retired->drain([&](uint64_t ptr, uint64_t bytes) {
        if (d.pool.give(ptr, bytes)) return;
        (void)hipFree((void*)ptr);
        d.device_bytes.fetch_sub((int64_t)(bytes < 4 ? 4 : bytes));
        d.frees.fetch_add(1);
    });
}

// Grows the activation scratch to at least `bytes`, waiting for the work
// that may still read the old one.
int ensure_scratch(Device& d, size_t bytes) {
    if (bytes <= d.act_scratch_bytes) return TMH_SUCCESS;
    size_t grown = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    hipError_t e = hipStreamSynchronize(d.stream);
    if (e != hipSuccess) return code(e);
    if (d.act_scratch) (void)hipFree(d.act_scratch);
    d.act_scratch = nullptr;
    d.act_scratch_bytes = 0;
    void* p = nullptr;
    e = device_malloc(&p, grown);
    if (e != hipSuccess) return e == hipErrorOutOfMemory ? TMH_ERROR_OUT_OF_MEMORY : code(e);
    d.act_scratch = (uint8_t*)p;
    d.act_scratch_bytes = grown;
    return TMH_SUCCESS;
}

size_t align256(size_t v) { return (v + 255u) & ~(size_t)255u; }

const char* library_name(int c) {
    switch (c) {
    case TMH_SUCCESS: return "TMH_SUCCESS";
    case TMH_ERROR_INVALID_VALUE: return "TMH_ERROR_INVALID_VALUE";
    case TMH_ERROR_SHAPE: return "TMH_ERROR_SHAPE";
    case TMH_ERROR_DTYPE: return "TMH_ERROR_DTYPE";
    case TMH_ERROR_NO_KERNELS: return "TMH_ERROR_NO_KERNELS";
    case TMH_ERROR_OUT_OF_MEMORY: return "TMH_ERROR_OUT_OF_MEMORY";
    case TMH_ERROR_EXECUTION: return "TMH_ERROR_EXECUTION";
    case TMH_ERROR_NO_DEVICE: return "TMH_ERROR_NO_DEVICE";
    case TMH_ERROR_BUSY: return "TMH_ERROR_BUSY";
    case TMH_ERROR_NOT_READY: return "TMH_ERROR_NOT_READY";
    case TMH_ERROR_SCRATCH_LIMIT: return "TMH_ERROR_SCRATCH_LIMIT";
    default: return nullptr;
    }
}

const char* library_string(int c) {
    switch (c) {
    case TMH_SUCCESS: return "no error";
    case TMH_ERROR_INVALID_VALUE: return "an argument is out of range";
    case TMH_ERROR_SHAPE: return "shapes do not agree";
    case TMH_ERROR_DTYPE: return "not a block format (Q8_0, Q4_0 or Q4_1)";
    case TMH_ERROR_NO_KERNELS: return "the library's kernels are not available";
    case TMH_ERROR_OUT_OF_MEMORY: return "out of device memory";
    case TMH_ERROR_EXECUTION: return "a kernel found an index out of range";
    case TMH_ERROR_NO_DEVICE: return "no such GPU";
    case TMH_ERROR_BUSY: return "the retired list is busy or full";
    case TMH_ERROR_NOT_READY: return "the device has not been set up: call tmh_init first";
    case TMH_ERROR_SCRATCH_LIMIT: return "the product's quantised activations exceed the fixed scratch (8 MiB)";
    default: return nullptr;
    }
}

}  // namespace

namespace tmh {

int device_context(DeviceContext* out, bool kernels) {
    if (kernels && g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    out->index = d->index;
    out->stream = d->stream;
    out->compute_units = d->compute_units;
    out->errors = d->errors;
    return TMH_SUCCESS;
}

void note_launch(int index, int ops, bool errors) {
    if (index < 0 || index >= MAX_DEVICES) return;
    Device& d = g_devices[index];
    if (errors) d.errors_pending.store(true);
    d.gpu_ops.fetch_add(ops);
}

}  // namespace tmh

extern "C" {

int tmh_init(int32_t* count) {
    if (!count) return TMH_ERROR_INVALID_VALUE;
    const int n = count_devices();
    // Sets every device up now (its stream, error buffer and the address of
    // its fixed scratch), so no later call needs to; the calling thread keeps
    // its device.
    const int keep = t_device;
    for (int i = 0; i < n; ++i) {
        t_device = i;
        int err;
        if (!current(&err)) {
            t_device = keep;
            return err;
        }
    }
    t_device = keep;
    if (n > 0 && keep >= 0 && keep < n) (void)hipSetDevice(keep);
    *count = n;
    return TMH_SUCCESS;
}

int tmh_device_info_get(int32_t device, tmh_device_info* out) {
    if (!out) return TMH_ERROR_INVALID_VALUE;
    if (device < 0 || device >= count_devices()) return TMH_ERROR_NO_DEVICE;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return code(e);
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    out->memory = prop.totalGlobalMem;
    out->compute_units = prop.multiProcessorCount;
    out->clock_khz = prop.clockRate;
    out->memory_clock_khz = prop.memoryClockRate;
    out->memory_bus_width = prop.memoryBusWidth;
    out->l2_bytes = prop.l2CacheSize;
    out->lds_bytes_per_block = (int32_t)prop.sharedMemPerBlock;
    return TMH_SUCCESS;
}

int tmh_set_device(int32_t device) {
    if (device < 0 || device >= count_devices()) return TMH_ERROR_NO_DEVICE;
    t_device = device;
    int err;
    current(&err);
    return err;
}

int tmh_get_device(int32_t* device) {
    if (!device) return TMH_ERROR_INVALID_VALUE;
    *device = t_device;
    return TMH_SUCCESS;
}

int tmh_malloc(uint64_t* ptr, uint64_t bytes) {
    if (!ptr) return TMH_ERROR_INVALID_VALUE;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    void* p = nullptr;
    const uint64_t size = bytes < 4 ? 4 : bytes;
    hipError_t e = device_malloc(&p, size);
    if (e == hipErrorOutOfMemory) return TMH_ERROR_OUT_OF_MEMORY;
    if (e != hipSuccess) return code(e);
    d->device_bytes.fetch_add((int64_t)size);
    *ptr = (uint64_t)p;
    return TMH_SUCCESS;
}

int tmh_free(uint64_t ptr) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if (ptr == 0) return TMH_SUCCESS;
    return code(hipFree((void*)ptr));
}

int tmh_free_any_thread(uint64_t ptr) {
    if (ptr) (void)hipFree((void*)ptr);
    return TMH_SUCCESS;
}

int tmh_upload(uint64_t dst, const void* src, uint64_t bytes) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    d->uploads.fetch_add(1);
    if (bytes == 0) return TMH_SUCCESS;
    if (!dst || !src) return TMH_ERROR_INVALID_VALUE;
    hipError_t e = hipMemcpyAsync((void*)dst, src, bytes, hipMemcpyHostToDevice, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    return code(e);
}

int tmh_upload_async(uint64_t dst, const void* src, uint64_t bytes) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    d->uploads.fetch_add(1);
    if (bytes == 0) return TMH_SUCCESS;
    if (!dst || !src) return TMH_ERROR_INVALID_VALUE;
    std::lock_guard<std::mutex> guard(d->staging_lock);
    Staging& s = d->staging;
    if (!s.ready) {
        for (int i = 0; i < Staging::SLOTS; ++i) {
            hipError_t e = hipHostMalloc(&s.slot[i], Staging::SLOT_BYTES, hipHostMallocDefault);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&s.done[i], hipEventDisableTiming);
            if (e != hipSuccess) return code(e);
        }
        s.ready = true;
    }
    uint64_t off = 0;
    while (off < bytes) {
        const size_t len = (size_t)std::min<uint64_t>(bytes - off, Staging::SLOT_BYTES);
        const int i = s.next;
        s.next = (s.next + 1) % Staging::SLOTS;
        if (s.used[i]) {
            hipError_t e = hipEventSynchronize(s.done[i]);
            if (e != hipSuccess) return code(e);
        }
        std::memcpy(s.slot[i], (const uint8_t*)src + off, len);
        hipError_t e = hipMemcpyAsync((void*)(dst + off), s.slot[i], len, hipMemcpyHostToDevice, d->stream);
        if (e == hipSuccess) e = hipEventRecord(s.done[i], d->stream);
        if (e != hipSuccess) return code(e);
        s.used[i] = true;
        off += len;
    }
    return TMH_SUCCESS;
}

int tmh_download(void* dst, uint64_t src, uint64_t bytes) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    d->downloads.fetch_add(1);
    if (bytes == 0) return TMH_SUCCESS;
    if (!dst || !src) return TMH_ERROR_INVALID_VALUE;
    hipError_t e = hipMemcpyAsync(dst, (const void*)src, bytes, hipMemcpyDeviceToHost, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    return code(e);
}

int tmh_copy(uint64_t dst, uint64_t src, uint64_t bytes) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if (bytes == 0) return TMH_SUCCESS;
    if (!dst || !src) return TMH_ERROR_INVALID_VALUE;
    return code(hipMemcpyAsync((void*)dst, (const void*)src, bytes, hipMemcpyDeviceToDevice, d->stream));
}

int tmh_synchronize(void) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    return code(hipStreamSynchronize(d->stream));
}

int tmh_alloc(uint64_t* ptr, uint64_t bytes) {
    if (!ptr) return TMH_ERROR_INVALID_VALUE;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    recycle_retired(*d);
    uint64_t p = d->pool.take(bytes);
    if (!p) {
        void* fresh = nullptr;
        const uint64_t size = bytes < 4 ? 4 : bytes;
        hipError_t e = device_malloc(&fresh, size);
        if (e == hipErrorOutOfMemory) return TMH_ERROR_OUT_OF_MEMORY;
        if (e != hipSuccess) return code(e);
        d->device_bytes.fetch_add((int64_t)size);
        p = (uint64_t)fresh;
    }
    *ptr = p;
    return TMH_SUCCESS;
}

int tmh_retire(uint64_t ptr, uint64_t bytes) {
    if (!ptr) return TMH_SUCCESS;
    int err;
    Device* d = current(&err);
    if (!d) {
        (void)hipFree((void*)ptr);
        return TMH_SUCCESS;
    }
    if (d->retired->push(ptr, bytes)) return TMH_SUCCESS;
    (void)hipFree((void*)ptr);
    d->device_bytes.fetch_sub((int64_t)(bytes < 4 ? 4 : bytes));
    d->frees.fetch_add(1);
    return TMH_SUCCESS;
}

int tmh_sync(void) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    hipError_t e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return code(e);
    recycle_retired(*d);
    if (d->errors_pending.exchange(false)) {
        int32_t got[3];
        e = hipMemcpy(got, d->errors, sizeof(got), hipMemcpyDeviceToHost);
        if (e != hipSuccess) return code(e);
        if (got[0] != 0) {
            {
                std::lock_guard<std::mutex> guard(d->report_lock);
                std::memcpy(d->report, got, sizeof(got));
            }
            e = hipMemset(d->errors, 0, sizeof(got));
            if (e != hipSuccess) return code(e);
            return TMH_ERROR_EXECUTION;
        }
    }
    return TMH_SUCCESS;
}

int tmh_pool_set_limit(int64_t bytes) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if (bytes < 0) return TMH_ERROR_INVALID_VALUE;
    d->pool.limit = bytes;
    return TMH_SUCCESS;
}

int tmh_counters_get(tmh_counters* out) {
    if (!out) return TMH_ERROR_INVALID_VALUE;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    out->uploads = d->uploads.load();
    out->downloads = d->downloads.load();
    out->gpu_ops = d->gpu_ops.load();
    out->device_bytes = d->device_bytes.load();
    out->pool_held = d->pool.held;
    out->pool_limit = d->pool.limit;
    out->pool_hits = d->pool.hits.load();
    out->pool_misses = d->pool.misses.load();
    out->frees = d->frees.load();
    out->launches = d->launches.load();
    return TMH_SUCCESS;
}

const char* tmh_error_name(int c) {
    if (const char* s = library_name(c)) return s;
    if (c > 0 && c < 1000) return hipGetErrorName((hipError_t)c);
    return "TMH_ERROR_UNKNOWN";
}

const char* tmh_error_string(int c) {
    if (const char* s = library_string(c)) return s;
    if (c > 0 && c < 1000) return hipGetErrorString((hipError_t)c);
    return "unknown error";
}

int tmh_error_report(int32_t out[3]) {
    if (!out) return TMH_ERROR_INVALID_VALUE;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    std::lock_guard<std::mutex> guard(d->report_lock);
    std::memcpy(out, d->report, sizeof(d->report));
    std::memset(d->report, 0, sizeof(d->report));
    return TMH_SUCCESS;
}

int tmh_debug_fail_allocations(int32_t count) {
    g_fail_allocations.store(count < 0 ? 0 : count);
    return TMH_SUCCESS;
}

int tmh_debug_disable_kernels(int32_t off) {
    g_kernels_off.store(off != 0);
    return TMH_SUCCESS;
}

int tmh_debug_f16_words(uint32_t first, uint32_t count, uint64_t dst) {
    if (g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if (count == 0) return TMH_SUCCESS;
    if (!dst || dst % 2u != 0 || (uint64_t)first + count > (1ull << 32)) return TMH_ERROR_INVALID_VALUE;
    hipError_t e = tmh::launch_f16_words(first, count, (uint16_t*)dst, d->stream);
    if (e == hipSuccess) d->gpu_ops.fetch_add(1);
    return code(e);
}

int tmh_debug_read(uint64_t src, uint64_t bytes, uint32_t workgroups, uint64_t out) {
    if (g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if (bytes == 0 || workgroups == 0) return TMH_SUCCESS;
    if (!src || !out || src % 16u != 0 || bytes % 16u != 0 || out % 4u != 0) return TMH_ERROR_INVALID_VALUE;
    hipError_t e = tmh::launch_read((const void*)src, bytes, workgroups, (uint32_t*)out, d->stream);
    if (e == hipSuccess) d->gpu_ops.fetch_add(1);
    return code(e);
}

int tmh_event_create(uint64_t* event) {
    if (!event) return TMH_ERROR_INVALID_VALUE;
    int err;
    if (!current(&err)) return err;
    hipEvent_t ev;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) return code(e);
    *event = (uint64_t)ev;
    return TMH_SUCCESS;
}

int tmh_event_record(uint64_t event) {
    int err;
    Device* d = current(&err);
    if (!d) return err;
    return code(hipEventRecord((hipEvent_t)event, d->stream));
}

int tmh_event_elapsed_ms(uint64_t start, uint64_t stop, float* ms) {
    if (!ms) return TMH_ERROR_INVALID_VALUE;
    hipError_t e = hipEventSynchronize((hipEvent_t)stop);
    if (e != hipSuccess) return code(e);
    return code(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
}

int tmh_event_destroy(uint64_t event) { return code(hipEventDestroy((hipEvent_t)event)); }

int tmh_quantize_rows_q8(uint64_t x, uint32_t rows, uint32_t k, uint32_t ldx, uint64_t scales, uint64_t sums,
                         uint64_t totals, uint64_t qs) {
    if (g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if (k == 0 || k % 32u != 0 || ldx < k) return TMH_ERROR_SHAPE;
    if (rows == 0) return TMH_SUCCESS;
    if (!x || !scales || !sums || !totals || !qs) return TMH_ERROR_INVALID_VALUE;
    if ((uint64_t)rows * k > 0x7fffffffull) return TMH_ERROR_SHAPE;
    hipError_t e = tmh::launch_quantize((const float*)x, ldx, rows, k, (float*)scales, (float*)sums, (int32_t*)totals,
                                        (int8_t*)qs, d->stream);
    if (e == hipSuccess) d->gpu_ops.fetch_add(1);
    return code(e);
}

namespace {

int check_product(uint32_t kind, uint32_t rows, uint32_t n, uint32_t k, uint32_t mode) {
    if (kind > 2u) return TMH_ERROR_DTYPE;
    if (k == 0 || k % 32u != 0) return TMH_ERROR_SHAPE;
    if (mode > TMH_MODE_MATRIX) return TMH_ERROR_INVALID_VALUE;
    if ((uint64_t)rows * n > 0x7fffffffull || (uint64_t)rows * k > 0x7fffffffull) return TMH_ERROR_SHAPE;
    return TMH_SUCCESS;
}

// The tiled one-row kernel (k_matvec_row, which quantises x itself) takes
// one-row AUTO products of at most this many weight bytes; larger ones run
// faster with each workgroup's weights staged into LDS at once (measured:
// Q4_1 8192x2048 one row 11.7 us against about 7; 2048x8192 21 against
// about 10).
constexpr uint64_t ROW_KERNEL_MAX_BYTES = 4ull << 20;

// AUTO products of one row above ROW_KERNEL_MAX_BYTES, and of two rows of
// k up to 2048: the one-row kernel with weights in LDS, which quantises x in
// every workgroup's prologue; where it does not fit, and for 2 to 8 rows:
// the few-rows kernel with weights in LDS, which does the same (k at most
// 2048), one launch and no scratch (measured, Q4_1 8192x2048: 7.4 / 8.1 /
// 9.0 us a call at 2 / 4 / 8 rows, against 8.2 / 9.8 / 9.8 for the quantise
// pass and the product).
// hipErrorInvalidValue, nothing launched, when the call is not for it.
// TMH_FEW_ROWS_KERNEL=lanes keeps the quantise pass and the lanes product,
// for comparisons.
// AUTO, or UNORDERED below the matrix cores' rows: the same kernels (UNORDERED
// folding in its own order).
bool auto_like(uint32_t mode) { return mode == TMH_MODE_AUTO || mode == TMH_MODE_UNORDERED; }

hipError_t few_rows_f32(const Device& d, uint32_t kind, const uint8_t* w, const float* x, uint32_t ldx, float* dst,
                        const float* bias, uint32_t rows, uint32_t n, uint32_t k, uint32_t mode) {
    static const bool lanes = [] {
        const char* env = getenv("TMH_FEW_ROWS_KERNEL");
        return env && strcmp(env, "lanes") == 0;
    }();
    const uint64_t bytes = (uint64_t)n * (k / 32u) * tmh::block_bytes(kind);
    if (lanes || !auto_like(mode) || rows > 8u || (rows == 1u && bytes <= ROW_KERNEL_MAX_BYTES))
        return hipErrorInvalidValue;
    // One row (k up to 8192), or two of k up to 2048: the one-row kernel
    // quantising x in its prologue (measured, Q4_1, one box: 8192x2048 one
    // row 5.35 us a call against 6.38 for the few-rows kernel, two rows 6.00
    // against 7.35; 2048x8192 one row 7.46 against 8.98 for the quantise pass
    // and the one-row kernel, two rows 10.85 against 10.66 for the quantise
    // pass and the lanes kernel, so not taken). TMH_ONE_F32=0 keeps the other
    // kernels, for comparisons.
    static const bool one_f32 = [] {
        const char* env = getenv("TMH_ONE_F32");
        return !(env && strcmp(env, "0") == 0);
    }();
    if (one_f32 && (rows == 1u || (rows == 2u && k <= 2048u))) {
        const hipError_t e =
            tmh::launch_product_f32_one(kind, w, x, ldx, dst, bias, rows, n, k, d.compute_units, d.stream);
        if (e != hipErrorInvalidValue) return e;
    }
    return tmh::launch_rows_product(kind, tmh::NB_F32, w, x, ldx, nullptr, 0.0f, tmh::Activations{}, dst, bias, 0u,
                                    rows, n, k, d.compute_units, d.stream);
}

}  // namespace

int tmh_block_matmul(uint32_t kind, uint64_t w, uint64_t w_byte_offset, uint64_t x, uint32_t ldx, uint64_t dst,
                     uint64_t bias, uint32_t rows, uint32_t n, uint32_t k, uint32_t mode) {
    if (g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    const tmh::TreeFold order(mode == TMH_MODE_UNORDERED);
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if ((err = check_product(kind, rows, n, k, mode)) != TMH_SUCCESS) return err;
    if (ldx < k) return TMH_ERROR_SHAPE;
    if (rows == 0 || n == 0) return TMH_SUCCESS;
    if (!w || !x || !dst) return TMH_ERROR_INVALID_VALUE;
    const uint8_t* wrow = (const uint8_t*)(w + w_byte_offset);
    // One row of a product of at most ROW_KERNEL_MAX_BYTES of weights: the
    // one-row kernel, which quantises x itself (one launch).
    if (rows == 1 && (!auto_like(mode) || (uint64_t)n * (k / 32u) * tmh::block_bytes(kind) <= ROW_KERNEL_MAX_BYTES) &&
        tmh::row_kernel_fits(mode, wrow, k)) {
        hipError_t e = tmh::launch_row(kind, wrow, (const float*)x, (float*)dst, (const float*)bias, n, k,
                                       d->compute_units, d->stream);
        if (e == hipSuccess) d->gpu_ops.fetch_add(1);
        return code(e);
    }
    hipError_t few = few_rows_f32(*d, kind, wrow, (const float*)x, ldx, (float*)dst, (const float*)bias, rows, n, k, mode);
    if (few != hipErrorInvalidValue) {
        if (few == hipSuccess) d->gpu_ops.fetch_add(1);
        return code(few);
    }
    std::lock_guard<std::mutex> guard(d->launch);
    if ((err = ensure_scratch(*d, scratch_need(rows, k))) != TMH_SUCCESS) return err;
    tmh::Activations act = tmh::carve_scratch(d->act_scratch, rows, k);
    hipError_t e = tmh::launch_quantize((const float*)x, ldx, rows, k, (float*)act.scales, (float*)act.sums,
                                        (int32_t*)act.totals, (int8_t*)act.qs, d->stream);
    if (e == hipSuccess)
        e = tmh::launch_block_matmul(kind, mode, (const uint8_t*)(w + w_byte_offset), act, (float*)dst,
                                     (const float*)bias, rows, n, k, d->compute_units, d->stream);
    if (e == hipSuccess) d->gpu_ops.fetch_add(1);
    return code(e);
}

int tmh_block_matmul_fixed(uint32_t kind, uint64_t w, uint64_t w_byte_offset, uint64_t x, uint32_t ldx, uint64_t dst,
                           uint64_t bias, uint32_t rows, uint32_t n, uint32_t k, uint32_t mode) {
    if (g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    const tmh::TreeFold order(mode == TMH_MODE_UNORDERED);
    const int n_devices = count_devices();
    if (n_devices == 0 || t_device < 0 || t_device >= n_devices) return TMH_ERROR_NO_DEVICE;
    Device* d = &g_devices[t_device];
    // Set-up allocates (a stream, the error buffer): it must have happened
    // in tmh_init or an earlier call, not here.
    if (!d->ready || !d->fixed_scratch) return TMH_ERROR_NOT_READY;
    int now = -1;
    if (hipGetDevice(&now) != hipSuccess || now != t_device) {
        hipError_t e = hipSetDevice(t_device);
        if (e != hipSuccess) return code(e);
    }
    int err;
    if ((err = check_product(kind, rows, n, k, mode)) != TMH_SUCCESS) return err;
    if (ldx < k) return TMH_ERROR_SHAPE;
    if (rows == 0 || n == 0) return TMH_SUCCESS;
    if (!w || !x || !dst) return TMH_ERROR_INVALID_VALUE;
    const uint8_t* wrow = (const uint8_t*)(w + w_byte_offset);
    // The same choice of kernels as tmh_block_matmul: a product that the
    // one-row or the few-rows kernel takes needs no scratch at all.
    if (rows == 1 && (!auto_like(mode) || (uint64_t)n * (k / 32u) * tmh::block_bytes(kind) <= ROW_KERNEL_MAX_BYTES) &&
        tmh::row_kernel_fits(mode, wrow, k)) {
        hipError_t e = tmh::launch_row(kind, wrow, (const float*)x, (float*)dst, (const float*)bias, n, k,
                                       d->compute_units, d->stream);
        if (e == hipSuccess) d->gpu_ops.fetch_add(1);
        return code(e);
    }
    hipError_t few = few_rows_f32(*d, kind, wrow, (const float*)x, ldx, (float*)dst, (const float*)bias, rows, n, k, mode);
    if (few != hipErrorInvalidValue) {
        if (few == hipSuccess) d->gpu_ops.fetch_add(1);
        return code(few);
    }
    if (scratch_need(rows, k) > TMH_FIXED_SCRATCH_BYTES) return TMH_ERROR_SCRATCH_LIMIT;
    // Calls share this device's array; the lock keeps each call's quantise
    // pass and product adjacent on the one stream, so they run in order.
    std::lock_guard<std::mutex> guard(d->fixed_launch);
    tmh::Activations act = tmh::carve_scratch(d->fixed_scratch, rows, k);
    hipError_t e = tmh::launch_quantize((const float*)x, ldx, rows, k, (float*)act.scales, (float*)act.sums,
                                        (int32_t*)act.totals, (int8_t*)act.qs, d->stream);
    if (e == hipSuccess)
        e = tmh::launch_block_matmul(kind, mode, wrow, act, (float*)dst, (const float*)bias, rows, n, k,
                                     d->compute_units, d->stream);
    if (e == hipSuccess) d->gpu_ops.fetch_add(1);
    return code(e);
}

int tmh_block_matmul_quantised(uint32_t kind, uint64_t w, uint64_t w_byte_offset, uint64_t scales, uint64_t sums,
                               uint64_t totals, uint64_t qs, uint64_t dst, uint64_t bias, uint32_t rows, uint32_t n,
                               uint32_t k, uint32_t mode) {
    if (g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if ((err = check_product(kind, rows, n, k, mode)) != TMH_SUCCESS) return err;
    if (rows == 0 || n == 0) return TMH_SUCCESS;
    if (!w || !scales || !sums || !totals || !qs || !dst) return TMH_ERROR_INVALID_VALUE;
    if (qs % 16u != 0 || scales % 8u != 0 || sums % 8u != 0 || totals % 8u != 0) return TMH_ERROR_INVALID_VALUE;
    const tmh::TreeFold order(mode == TMH_MODE_UNORDERED);
    tmh::Activations act{(const float*)scales, (const float*)sums, (const int32_t*)totals, (const int8_t*)qs};
    hipError_t e = tmh::launch_block_matmul(kind, mode, (const uint8_t*)(w + w_byte_offset), act, (float*)dst,
                                            (const float*)bias, rows, n, k, d->compute_units, d->stream);
    if (e == hipSuccess) d->gpu_ops.fetch_add(1);
    return code(e);
}

int tmh_gather_blocks(uint32_t kind, uint64_t table, uint64_t table_byte_offset, int32_t table_rows, uint32_t width,
                      uint64_t ids, uint32_t count, uint64_t dst) {
    if (g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    if (kind > 2u) return TMH_ERROR_DTYPE;
    if (width == 0 || width % 32u != 0 || table_rows < 0) return TMH_ERROR_SHAPE;
    if ((uint64_t)count * width > 0x7fffffffull) return TMH_ERROR_SHAPE;
    if (count == 0) return TMH_SUCCESS;
    if (!table || !ids || !dst) return TMH_ERROR_INVALID_VALUE;
    d->errors_pending.store(true);
    hipError_t e = tmh::launch_gather(kind, (const uint8_t*)(table + table_byte_offset), table_rows, width,
                                      (const int32_t*)ids, count, (float*)dst, d->errors, d->stream);
    if (e == hipSuccess) d->gpu_ops.fetch_add(1);
    return code(e);
}

namespace {

// A plan runs the streamed kernel (`stream`, device memory `mem` holding its
// product table and workgroup starts) or, where its products do not fit
// that kernel, the tiled one-row kernel (`table`, then each tile's product
// index in `owner`).
struct Plan {
    int device;
    uint32_t kind;
    uint32_t count;
    uint32_t tiles;
    size_t act_bytes, part_bytes;
    tmh::RowProduct* table;
    uint32_t* owner;
    bool streamed;
    tmh::StreamLaunch stream;
    void* mem;
    uint32_t mode = TMH_MODE_AUTO;  // AUTO, or UNORDERED (tmh_plan_set_mode)
};

// Builds the streamed form of a plan; false (nothing allocated) when the
// products do not fit the streamed kernel or TMH_PLAN_KERNEL=rows asks for
// the tiled one.
int stream_plan(Plan* p, const tmh_product* given, const std::vector<tmh::RowProduct>& rows, int compute_units,
                bool& made) {
    made = false;
    const char* env = getenv("TMH_PLAN_KERNEL");
    if (env && std::string(env) == "rows") return TMH_SUCCESS;
    std::vector<tmh::StreamProduct> products(rows.size());
    for (size_t i = 0; i < rows.size(); ++i) {
        tmh::StreamProduct& q = products[i];
        const tmh_product& g = given[i];
        q = tmh::StreamProduct{};
        q.w = rows[i].w, q.x = rows[i].x, q.dst = rows[i].dst, q.bias = rows[i].bias;
        q.n = rows[i].n, q.k = rows[i].k;
        q.mode = g.x_mode, q.eps = g.eps;
        if (g.x_mode == TMH_X_RMSNORM) q.aux0 = (const float*)g.norm;
        if (g.x_mode == TMH_X_QUANTISED) {
            q.aux0 = (const float*)g.scales;
            q.aux1 = p->kind == 1u ? (const void*)g.totals : p->kind == 2u ? (const void*)g.sums : nullptr;
        }
    }
    tmh::StreamLaunch l{};
    void* mem = nullptr;
    const hipError_t e = tmh::make_stream(p->kind, products, compute_units, l, &mem);
    if (e == hipErrorInvalidValue) return TMH_SUCCESS;  // not for the streamed kernel
    if (e != hipSuccess) return e == hipErrorOutOfMemory ? TMH_ERROR_OUT_OF_MEMORY : code(e);
    p->stream = l;
    p->mem = mem;
    p->streamed = true;
    made = true;
    return TMH_SUCCESS;
}

}  // namespace

int tmh_plan_create(uint32_t kind, const tmh_product* products, uint32_t count, uint64_t* plan) {
    if (!plan || (count && !products)) return TMH_ERROR_INVALID_VALUE;
    if (kind > 2u) return TMH_ERROR_DTYPE;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    std::vector<tmh::RowProduct> rows(count);
    uint32_t first = 0;
    size_t act_bytes = 0, part_bytes = 0;
    bool modes = false;  // a product whose x is not plain f32: the streamed kernel only
    for (uint32_t i = 0; i < count; ++i) {
        const tmh_product& q = products[i];
        if (q.k == 0 || q.k % 32u != 0 || q.n == 0) return TMH_ERROR_SHAPE;
        if (!q.w || !q.x || !q.dst) return TMH_ERROR_INVALID_VALUE;
        if (q.x_mode > TMH_X_QUANTISED) return TMH_ERROR_INVALID_VALUE;
        if (q.x_mode == TMH_X_RMSNORM && !q.norm) return TMH_ERROR_INVALID_VALUE;
        if (q.x_mode == TMH_X_QUANTISED && (!q.scales || (kind == 1u && !q.totals) || (kind == 2u && !q.sums)))
            return TMH_ERROR_INVALID_VALUE;
        modes = modes || q.x_mode != TMH_X_F32;
        const uint8_t* w = (const uint8_t*)(q.w + q.w_byte_offset);
        if (!tmh::row_kernel_fits(TMH_MODE_LANES, w, q.k)) return TMH_ERROR_SHAPE;
        tmh::RowProduct& r = rows[i];
        r.w = w;
        r.x = (const float*)q.x;
        r.dst = (float*)q.dst;
        r.bias = (const float*)q.bias;
        r.n = q.n;
        r.k = q.k;
        tmh::plan_row(kind, r, d->compute_units);
        r.first = first;
        if ((uint64_t)first + r.tiles > 0x7fffffffull) return TMH_ERROR_SHAPE;
        first += r.tiles;
        act_bytes = std::max(act_bytes, tmh::row_act_bytes(r));
        part_bytes = std::max(part_bytes, tmh::row_part_bytes(r));
    }
    Plan* p = new Plan{d->index, kind, count, first, act_bytes, part_bytes, nullptr, nullptr, false, {}, nullptr};
    if (count) {
        bool made = false;
        const int r = stream_plan(p, products, rows, d->compute_units, made);
        if (r != TMH_SUCCESS) {
            delete p;
            return r;
        }
        if (made) {
            *plan = (uint64_t)p;
            return TMH_SUCCESS;
        }
    }
    if (modes) {
        delete p;
        return TMH_ERROR_SHAPE;
    }
    if (act_bytes + part_bytes > 64u * 1024u) {
        delete p;
        return TMH_ERROR_SHAPE;
    }
    if (count) {
        // One allocation: the product table, then the tile -> product map.
        std::vector<uint32_t> owner(first);
        for (uint32_t i = 0; i < count; ++i)
            for (uint32_t t = 0; t < rows[i].tiles; ++t) owner[rows[i].first + t] = i;
        const size_t table_bytes = align256(sizeof(tmh::RowProduct) * count);
        void* mem = nullptr;
        hipError_t e = device_malloc(&mem, table_bytes + sizeof(uint32_t) * first);
        if (e == hipSuccess) e = hipMemcpy(mem, rows.data(), sizeof(tmh::RowProduct) * count, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy((uint8_t*)mem + table_bytes, owner.data(), sizeof(uint32_t) * first, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            if (mem) (void)hipFree(mem);
            delete p;
            return e == hipErrorOutOfMemory ? TMH_ERROR_OUT_OF_MEMORY : code(e);
        }
        p->table = (tmh::RowProduct*)mem;
        p->owner = (uint32_t*)((uint8_t*)mem + table_bytes);
    }
    *plan = (uint64_t)p;
    return TMH_SUCCESS;
}

int tmh_plan_run(uint64_t plan) {
    if (g_kernels_off.load()) return TMH_ERROR_NO_KERNELS;
    if (!plan) return TMH_ERROR_INVALID_VALUE;
    int err;
    Device* d = current(&err);
    if (!d) return err;
    Plan* p = (Plan*)plan;
    if (p->device != d->index) return TMH_ERROR_INVALID_VALUE;
    const tmh::TreeFold order(p->mode == TMH_MODE_UNORDERED);
    hipError_t e = p->streamed ? tmh::launch_stream(p->kind, p->stream, d->stream)
                               : tmh::launch_rows(p->kind, p->table, p->owner, p->tiles, p->act_bytes,
                                                  p->part_bytes, d->compute_units, d->stream);
    if (e == hipSuccess) d->gpu_ops.fetch_add(p->count);
    return code(e);
}

int tmh_plan_set_mode(uint64_t plan, uint32_t mode) {
    if (!plan || (mode != TMH_MODE_AUTO && mode != TMH_MODE_UNORDERED)) return TMH_ERROR_INVALID_VALUE;
    ((Plan*)plan)->mode = mode;
    return TMH_SUCCESS;
}

int tmh_plan_describe(uint64_t plan, char* text, uint32_t size) {
    if (!plan || !text || size == 0) return TMH_ERROR_INVALID_VALUE;
    const Plan* p = (const Plan*)plan;
    if (p->streamed)
        snprintf(text, size, "tmh::k_matvec_stream<%u, %u, %s> grid %u, LDS %zu B, %u steps of up to %u B",
                 p->kind, p->stream.ring, p->stream.has_bias ? "true" : "false", p->stream.grid, p->stream.lds,
                 p->stream.total, 8192u);
    else
        snprintf(text, size, "tmh::k_matvec_rows<%u> %u tiles, LDS %zu B", p->kind, p->tiles,
                 p->act_bytes + p->part_bytes);
    return TMH_SUCCESS;
}

int tmh_plan_destroy(uint64_t plan) {
    if (!plan) return TMH_SUCCESS;
    Plan* p = (Plan*)plan;
    int err;
    Device* d = current(&err);
    if (d) (void)hipStreamSynchronize(d->stream);
    if (p->table) (void)hipFree(p->table);
    if (p->mem) (void)hipFree(p->mem);
    delete p;
    return TMH_SUCCESS;
}

}  // extern "C"
