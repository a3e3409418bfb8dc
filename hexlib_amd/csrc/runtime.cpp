// Library state (current stream, launch errors) and the batch session:
// open/start/mmap/invoke/stop/close, the GPU counterpart of the reference's
// FastRPC skel (hexlib/runtime/skel/skel.c:30-197, skel_dispatch.c:80-302,
// skel_bufs.c:136-230).
//
// Validation and tensor resolution are pure host code that returns a status
// before any HIP call, so every refusal is testable without a GPU (DRYRUN
// invokes never touch the device). Status OK is 1 and the response header is
// written as ERR_INTERNAL first, so an unwritten or half-written response
// never reads as success.
//
// Beyond the reference's checks, each tensor's element extent (ne) must fit
// its declared byte count, and the generated entries check every buffer
// against the extent the kernel will touch: a malformed blob is refused, it
// never becomes an out-of-bounds GPU access.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "hexlib_gpu.h"
#include "internal.h"

namespace hx {

// Per host thread: two threads (say, two sessions invoked concurrently) never
// launch on each other's stream or take each other's launch errors.
static thread_local hipStream_t t_stream = nullptr;
static thread_local int t_error = 0;
static thread_local bool t_dry_run = false;

hipStream_t stream() { return t_stream; }

void note(hipError_t e) {
    if (e != hipSuccess && t_error == 0) t_error = (int) e;
}

bool dry_run() { return t_dry_run; }
void set_dry_run(bool on) { t_dry_run = on; }

// ---- scratch ----

constexpr int MAX_DEVICES = 16;

struct Scratch {
    std::mutex mu;
    void *ptr[MAX_DEVICES] = {};
    size_t size[MAX_DEVICES] = {};
    // buffers replaced by a larger one: a graph captured earlier may still
    // read them, so they live until the scratch is freed
    std::vector<void *> retired;
};

static Scratch g_default_scratch;
static thread_local Scratch *t_scratch = nullptr;
static thread_local size_t t_reserve = 0;
static thread_local float *t_fixed_ptr = nullptr;
static thread_local size_t t_fixed_cap = 0;
static thread_local bool t_fixed_on = false, t_fixed_refused = false;

Scratch *scratch_new() { return new (std::nothrow) Scratch(); }

void scratch_free(Scratch *s) {
    if (!s) return;
    for (int d = 0; d < MAX_DEVICES; ++d)
        if (s->ptr[d]) hipFree(s->ptr[d]);
    for (void *p : s->retired) hipFree(p);
    delete s;
}

Scratch *current_scratch() { return t_scratch ? t_scratch : &g_default_scratch; }
void set_current_scratch(Scratch *s) { t_scratch = s; }

static int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= MAX_DEVICES) d = 0;
    return d;
}

float *workspace(size_t bytes) {
    if (t_fixed_on) {
        if (bytes <= t_fixed_cap) return t_fixed_ptr;
        t_fixed_refused = true;
        return nullptr;
    }
    Scratch *s = current_scratch();
    const int d = current_device();
    std::lock_guard<std::mutex> g(s->mu);
    if (s->size[d] >= bytes) return static_cast<float *>(s->ptr[d]);
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream(), &st) != hipSuccess || st != hipStreamCaptureStatusNone)
        return nullptr;
    void *p = nullptr;
    const size_t sz = bytes < ((size_t) 64 << 20) ? ((size_t) 64 << 20) : bytes;
    if (hipMalloc(&p, sz) != hipSuccess) return nullptr;
    if (s->ptr[d]) s->retired.push_back(s->ptr[d]);
    s->ptr[d] = p;
    s->size[d] = sz;
    return static_cast<float *>(p);
}

void reserve_workspace(size_t bytes) {
    if (bytes > t_reserve) t_reserve = bytes;
}

int prepare_workspace() {
    const size_t want = t_reserve;
    t_reserve = 0;
    if (!want) return 0;
    return workspace(want) ? 0 : -1;
}

FixedWorkspace::FixedWorkspace(float *ptr, size_t cap) {
    t_fixed_ptr = ptr;
    t_fixed_cap = cap;
    t_fixed_on = true;
    t_fixed_refused = false;
}
FixedWorkspace::~FixedWorkspace() {
    t_fixed_on = false;
    t_fixed_ptr = nullptr;
    t_fixed_cap = 0;
}
bool FixedWorkspace::refused() { return t_fixed_refused; }

}  // namespace hx

extern "C" {

void hexlib_gpu_set_stream(void *stream) { hx::t_stream = (hipStream_t) stream; }
void *hexlib_gpu_get_stream(void) { return (void *) hx::t_stream; }
int hexlib_gpu_take_error(void) {
    const int e = hx::t_error;
    hx::t_error = 0;
    return e;
}
const char *hexlib_gpu_error_string(int e) { return hipGetErrorString((hipError_t) e); }

const char *hexlib_gpu_status_name(int s) {
    switch (s) {
    case HEXLIB_DSP_OK: return "OK";
    case HEXLIB_DSP_ERR_INTERNAL: return "ERR_INTERNAL";
    case HEXLIB_DSP_ERR_BAD_MAGIC: return "ERR_BAD_MAGIC";
    case HEXLIB_DSP_ERR_BAD_VERSION: return "ERR_BAD_VERSION";
    case HEXLIB_DSP_ERR_TRUNCATED: return "ERR_TRUNCATED";
    case HEXLIB_DSP_ERR_INVAL_PARAMS: return "ERR_INVAL_PARAMS";
    case HEXLIB_DSP_ERR_UNMAPPED: return "ERR_UNMAPPED";
    case HEXLIB_DSP_ERR_NO_MMAP_SLOT: return "ERR_NO_MMAP_SLOT";
    case HEXLIB_DSP_ERR_MMAP_FAILED: return "ERR_MMAP_FAILED";
    case HEXLIB_DSP_ERR_NO_KERNEL: return "ERR_NO_KERNEL";
    case HEXLIB_DSP_ERR_VTCM_TOO_SMALL: return "ERR_VTCM_TOO_SMALL";
    case HEXLIB_DSP_ERR_VTCM_RECLAIMED: return "ERR_VTCM_RECLAIMED";
    case HEXLIB_DSP_ERR_REQUIRES: return "ERR_REQUIRES";
    case HEXLIB_DSP_ERR_NOT_STARTED: return "ERR_NOT_STARTED";
    case HEXLIB_DSP_ERR_CACHE: return "ERR_CACHE";
    default: return "UNKNOWN";
    }
}

uint32_t hexlib_gpu_struct_sizes(uint32_t *out, uint32_t cap) {
    const uint32_t sizes[] = {
        (uint32_t) sizeof(struct hexlib_batch_hdr),  (uint32_t) sizeof(struct hexlib_buf_desc),
        (uint32_t) sizeof(struct hexlib_tensor),     (uint32_t) sizeof(struct hexlib_op_desc),
        (uint32_t) sizeof(struct hexlib_batch_rsp_hdr), (uint32_t) sizeof(struct hexlib_op_result),
        (uint32_t) sizeof(hexlib_args),
    };
    const uint32_t n = sizeof(sizes) / sizeof(sizes[0]);
    for (uint32_t i = 0; i < n && i < cap; ++i) out[i] = sizes[i];
    return n;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// session

struct hexlib_gpu_ctx {
    struct Slot {
        void *base;
        uint64_t size;
        int64_t fd;  // -1 = free
    };
    Slot mmap[HEXLIB_MAX_MMAPS];
    uint64_t map_generation = 0;  // bumps on every mmap/munmap: invalidates graphs
    int started = 0;
    uint32_t sess_id = 0;
    int device = 0;
    uint64_t max_vmem = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;

    // working copies of the current blob (reference: static, non-reentrant;
    // here per session and guarded by `mu`)
    hexlib_buf_desc bufs[HEXLIB_MAX_BUFS];
    void *buf_base[HEXLIB_MAX_BUFS];
    hexlib_tensor tens[HEXLIB_MAX_TENSORS];
    void *tdata[HEXLIB_MAX_TENSORS];

    // one cached graph: the blob it was captured from and the mapping epoch
    std::vector<uint8_t> graph_blob;
    uint64_t graph_generation = 0;
    hipGraphExec_t graph_exec = nullptr;
    uint32_t graph_nops = 0;

    std::vector<hipEvent_t> events;

    // this session's split-K workspace (never shared with another session)
    hx::Scratch *scratch = nullptr;
};

namespace {

constexpr uint32_t ARCH = 950;

void write_hdr(uint8_t *rsp, uint32_t status, uint32_t n_ops, uint64_t cycles) {
    hexlib_batch_rsp_hdr h;
    std::memset(&h, 0, sizeof(h));
    h.magic = HEXLIB_BATCH_MAGIC;
    h.version = HEXLIB_BATCH_VERSION;
    h.status = status;
    h.n_ops = n_ops;
    h.cycles_total = cycles;
    h.arch = ARCH;
    std::memcpy(rsp, &h, sizeof(h));
}

hexlib_gpu_ctx::Slot *find_fd(hexlib_gpu_ctx *ctx, uint32_t fd) {
    for (auto &m : ctx->mmap)
        if (m.size && m.fd == (int64_t) fd) return &m;
    return nullptr;
}

bool elem_capacity_ok(const hexlib_tensor &t) {
    // True if ne fits nbytes for the declared dtype. The element count is a
    // product of four uint32 factors, each widened before its multiply (the
    // product stays below 2^128); it is compared against nbytes divided by the
    // element size, so no side of the comparison can wrap.
    typedef unsigned __int128 u128;
    const u128 n = (u128) t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    const u128 nb = t.nbytes;
    switch (t.dtype) {
    case HEXLIB_DTYPE_FP32:
    case HEXLIB_DTYPE_INT32: return n <= nb / 4;
    case HEXLIB_DTYPE_FP16: return n <= nb / 2;
    case HEXLIB_DTYPE_Q4_0: return n % 32 == 0 && n / 32 <= nb / 18;
    case HEXLIB_DTYPE_Q8_0: return n % 32 == 0 && n / 32 <= nb / 34;
    default: return false;
    }
}

const hexlib_kernel_entry *find_kernel(uint32_t kind) {
    for (uint32_t j = 0; j < hexlib_kernel_table_len; ++j)
        if (hexlib_kernel_table[j].kind == kind) return &hexlib_kernel_table[j];
    return nullptr;
}

// Header + section bounds + response room: skel_dispatch.c:94-132.
int validate_header(const uint8_t *batch, uint32_t len, uint32_t rsp_cap, hexlib_batch_hdr &hdr) {
    if (len < sizeof(hexlib_batch_hdr)) return HEXLIB_DSP_ERR_TRUNCATED;
    std::memcpy(&hdr, batch, sizeof(hdr));
    if (hdr.magic != HEXLIB_BATCH_MAGIC) return HEXLIB_DSP_ERR_BAD_MAGIC;
    if (hdr.version != HEXLIB_BATCH_VERSION) return HEXLIB_DSP_ERR_BAD_VERSION;
    if (hdr.total_size != len) return HEXLIB_DSP_ERR_TRUNCATED;
    if (hdr.n_bufs > HEXLIB_MAX_BUFS || hdr.n_tensors > HEXLIB_MAX_TENSORS)
        return HEXLIB_DSP_ERR_INVAL_PARAMS;
    if ((uint64_t) hdr.off_bufs + (uint64_t) hdr.n_bufs * sizeof(hexlib_buf_desc) > len ||
        (uint64_t) hdr.off_tensors + (uint64_t) hdr.n_tensors * sizeof(hexlib_tensor) > len ||
        (uint64_t) hdr.off_ops + (uint64_t) hdr.n_ops * sizeof(hexlib_op_desc) > len)
        return HEXLIB_DSP_ERR_TRUNCATED;
    if ((uint64_t) sizeof(hexlib_batch_rsp_hdr) + (uint64_t) hdr.n_ops * sizeof(hexlib_op_result) >
        rsp_cap)
        return HEXLIB_DSP_ERR_TRUNCATED;
    return HEXLIB_DSP_OK;
}

// fd -> registered base, then every tensor -> base + offset (skel_bufs.c:136-185).
int resolve(hexlib_gpu_ctx *ctx, const uint8_t *batch, const hexlib_batch_hdr &hdr) {
    std::memcpy(ctx->bufs, batch + hdr.off_bufs, hdr.n_bufs * sizeof(hexlib_buf_desc));
    std::memcpy(ctx->tens, batch + hdr.off_tensors, hdr.n_tensors * sizeof(hexlib_tensor));
    for (uint32_t i = 0; i < hdr.n_bufs; ++i) {
        hexlib_buf_desc &b = ctx->bufs[i];
        b.base = 0;  // whatever the host wrote is never used
        ctx->buf_base[i] = nullptr;
        hexlib_gpu_ctx::Slot *m = find_fd(ctx, b.fd);
        if (!m) return HEXLIB_DSP_ERR_UNMAPPED;
        if (b.size > m->size) return HEXLIB_DSP_ERR_INVAL_PARAMS;
        ctx->buf_base[i] = m->base;
    }
    for (uint32_t i = 0; i < hdr.n_tensors; ++i) {
        const hexlib_tensor &t = ctx->tens[i];
        if (t.bi >= hdr.n_bufs) return HEXLIB_DSP_ERR_INVAL_PARAMS;
        if (!ctx->buf_base[t.bi]) return HEXLIB_DSP_ERR_UNMAPPED;
        if ((uint64_t) t.offset + (uint64_t) t.nbytes > ctx->bufs[t.bi].size)
            return HEXLIB_DSP_ERR_TRUNCATED;
        if (!elem_capacity_ok(t)) return HEXLIB_DSP_ERR_INVAL_PARAMS;
        ctx->tdata[i] = static_cast<uint8_t *>(ctx->buf_base[t.bi]) + t.offset;
    }
    return HEXLIB_DSP_OK;
}

// Builds hexlib_args for op i (src then dst, skel_dispatch.c:209-248).
int build_args(hexlib_gpu_ctx *ctx, const hexlib_batch_hdr &hdr, const hexlib_op_desc &op,
               hexlib_args &a) {
    std::memset(&a, 0, sizeof(a));
    uint32_t nb = 0;
    for (uint32_t s = 0; s < HEXLIB_MAX_SRC + HEXLIB_MAX_DST; ++s) {
        const uint16_t ti = s < HEXLIB_MAX_SRC ? op.src[s] : op.dst[s - HEXLIB_MAX_SRC];
        if (ti == HEXLIB_NO_TENSOR) continue;
        if (ti >= hdr.n_tensors || nb >= HEXLIB_MAX_BUFS) return HEXLIB_DSP_ERR_INVAL_PARAMS;
        const hexlib_tensor &t = ctx->tens[ti];
        a.buf[nb] = ctx->tdata[ti];
        a.dtype[nb] = t.dtype;
        a.layout[nb] = t.layout;
        for (int e = 0; e < 4; ++e) a.ne[nb][e] = t.ne[e];
        ++nb;
    }
    a.n_buf = nb;
    a.vtcm = nullptr;
    a.vtcm_size = 0;
    a.params = op.params;
    a.n_threads = 1;
    return HEXLIB_DSP_OK;
}

int ensure_events(hexlib_gpu_ctx *ctx, size_t n) {
    while (ctx->events.size() < n) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return HEXLIB_DSP_ERR_INTERNAL;
        ctx->events.push_back(e);
    }
    return HEXLIB_DSP_OK;
}

void drop_graph(hexlib_gpu_ctx *ctx) {
    if (ctx->graph_exec) hipGraphExecDestroy(ctx->graph_exec);
    ctx->graph_exec = nullptr;
    ctx->graph_blob.clear();
    ctx->graph_nops = 0;
}

// Runs ops [0, n) through their entries on the library stream. Per-op results
// are pre-filled with ERR_INTERNAL; stops at the first failing op.
int run_ops(hexlib_gpu_ctx *ctx, const uint8_t *batch, const hexlib_batch_hdr &hdr,
            hexlib_op_result *results, uint32_t &done, bool timed) {
    int status = HEXLIB_DSP_OK;
    done = 0;
    for (uint32_t i = 0; i < hdr.n_ops; ++i) {
        hexlib_op_desc op;
        std::memcpy(&op, batch + hdr.off_ops + (uint64_t) i * sizeof(op), sizeof(op));
        results[i].kind = op.kind;
        results[i].status = HEXLIB_DSP_ERR_INTERNAL;
        results[i].cycles = 0;
        done = i + 1;
        const hexlib_kernel_entry *k = find_kernel(op.kind);
        if (!k) {
            results[i].status = HEXLIB_DSP_ERR_NO_KERNEL;
            status = HEXLIB_DSP_ERR_NO_KERNEL;
            break;
        }
        hexlib_args a;
        int rc = build_args(ctx, hdr, op, a);
        if (rc != HEXLIB_DSP_OK) {
            results[i].status = (uint32_t) rc;
            status = rc;
            break;
        }
        if (timed) hipEventRecord(ctx->events[2 * i], ctx->stream);
        rc = k->fn(&a);
        if (timed) hipEventRecord(ctx->events[2 * i + 1], ctx->stream);
        results[i].status = (uint32_t) rc;
        if (rc != HEXLIB_DSP_OK) {
            status = rc;
            break;
        }
    }
    return status;
}

struct StreamScope {
    void *saved;
    explicit StreamScope(hipStream_t s) : saved(hexlib_gpu_get_stream()) { hexlib_gpu_set_stream(s); }
    ~StreamScope() { hexlib_gpu_set_stream(saved); }
};

struct ScratchScope {
    hx::Scratch *saved;
    explicit ScratchScope(hx::Scratch *s) : saved(hx::current_scratch()) { hx::set_current_scratch(s); }
    ~ScratchScope() { hx::set_current_scratch(saved); }
};

struct DryScope {
    bool saved;
    explicit DryScope(bool on) : saved(hx::dry_run()) { hx::set_dry_run(on); }
    ~DryScope() { hx::set_dry_run(saved); }
};

}  // namespace

extern "C" {

int hexlib_gpu_open(hexlib_gpu_ctx **out) {
    if (!out) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    hexlib_gpu_ctx *ctx = new (std::nothrow) hexlib_gpu_ctx();
    if (!ctx) return HEXLIB_DSP_ERR_INTERNAL;
    ctx->scratch = hx::scratch_new();
    if (!ctx->scratch) {
        delete ctx;
        return HEXLIB_DSP_ERR_INTERNAL;
    }
    for (auto &m : ctx->mmap) {
        m.base = nullptr;
        m.size = 0;
        m.fd = -1;
    }
    *out = ctx;
    return HEXLIB_DSP_OK;
}

int hexlib_gpu_start(hexlib_gpu_ctx *ctx, uint32_t sess_id, int device, uint64_t max_vmem) {
    if (!ctx) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (ctx->started) return HEXLIB_DSP_OK;
    if (hipSetDevice(device) != hipSuccess) return HEXLIB_DSP_ERR_INTERNAL;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess)
        return HEXLIB_DSP_ERR_INTERNAL;
    ctx->sess_id = sess_id;
    ctx->device = device;
    ctx->max_vmem = max_vmem;
    ctx->started = 1;
    return HEXLIB_DSP_OK;
}

int hexlib_gpu_stop(hexlib_gpu_ctx *ctx) {
    if (!ctx) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (!ctx->started) return HEXLIB_DSP_OK;
    hipStreamSynchronize(ctx->stream);
    drop_graph(ctx);
    for (hipEvent_t e : ctx->events) hipEventDestroy(e);
    ctx->events.clear();
    hipStreamDestroy(ctx->stream);
    ctx->stream = nullptr;
    ctx->started = 0;
    return HEXLIB_DSP_OK;
}

int hexlib_gpu_close(hexlib_gpu_ctx *ctx) {
    if (!ctx) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    hexlib_gpu_stop(ctx);   // drains the session stream first
    hx::scratch_free(ctx->scratch);
    delete ctx;
    return HEXLIB_DSP_OK;
}

int hexlib_gpu_mmap(hexlib_gpu_ctx *ctx, uint32_t fd, void *dev_ptr, uint64_t size) {
    if (!ctx || !dev_ptr || !size) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (hexlib_gpu_ctx::Slot *m = find_fd(ctx, fd)) {
        // Re-registering an fd is idempotent only for the same memory.
        return (m->base == dev_ptr && m->size == size) ? HEXLIB_DSP_OK : HEXLIB_DSP_ERR_MMAP_FAILED;
    }
    for (auto &m : ctx->mmap) {
        if (m.size) continue;
        m.base = dev_ptr;
        m.size = size;
        m.fd = fd;
        ++ctx->map_generation;
        return HEXLIB_DSP_OK;
    }
    return HEXLIB_DSP_ERR_NO_MMAP_SLOT;
}

int hexlib_gpu_munmap(hexlib_gpu_ctx *ctx, uint32_t fd) {
    if (!ctx) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    std::lock_guard<std::mutex> g(ctx->mu);
    hexlib_gpu_ctx::Slot *m = find_fd(ctx, fd);
    if (!m) return HEXLIB_DSP_ERR_UNMAPPED;
    m->base = nullptr;
    m->size = 0;
    m->fd = -1;
    ++ctx->map_generation;
    return HEXLIB_DSP_OK;
}

int hexlib_gpu_hwinfo(hexlib_gpu_ctx *ctx, uint32_t *arch, uint32_t *n_cu, uint32_t *n_threads,
                      uint64_t *lds_per_cu) {
    if (!ctx || !arch || !n_cu || !n_threads || !lds_per_cu) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    if (!ctx->started) return HEXLIB_DSP_ERR_NOT_STARTED;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, ctx->device) != hipSuccess) return HEXLIB_DSP_ERR_INTERNAL;
    *arch = ARCH;
    *n_cu = (uint32_t) prop.multiProcessorCount;
    *n_threads = 1;
    *lds_per_cu = (uint64_t) prop.maxSharedMemoryPerMultiProcessor;
    return HEXLIB_DSP_OK;
}

void *hexlib_gpu_session_stream(hexlib_gpu_ctx *ctx) { return ctx ? (void *) ctx->stream : nullptr; }

int hexlib_gpu_invoke(hexlib_gpu_ctx *ctx, const uint8_t *batch, uint32_t len, uint8_t *rsp,
                      uint32_t rsp_cap, uint32_t *rsp_len, uint32_t flags) {
    if (!rsp_len) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    *rsp_len = 0;
    if (!rsp || rsp_cap < sizeof(hexlib_batch_rsp_hdr)) return HEXLIB_DSP_ERR_TRUNCATED;
    write_hdr(rsp, HEXLIB_DSP_ERR_INTERNAL, 0, 0);
    *rsp_len = sizeof(hexlib_batch_rsp_hdr);
    if (!ctx || (!batch && len)) {
        write_hdr(rsp, HEXLIB_DSP_ERR_INVAL_PARAMS, 0, 0);
        return HEXLIB_DSP_ERR_INVAL_PARAMS;
    }
    std::lock_guard<std::mutex> g(ctx->mu);
    const bool dry = flags & HEXLIB_GPU_INVOKE_DRYRUN;
    const bool timed = !dry && (flags & HEXLIB_GPU_INVOKE_TIMED);
    const bool use_graph = !dry && (flags & HEXLIB_GPU_INVOKE_GRAPH);
    const bool sync = !(flags & HEXLIB_GPU_INVOKE_NOSYNC);
    if (!ctx->started && !dry) {
        write_hdr(rsp, HEXLIB_DSP_ERR_NOT_STARTED, 0, 0);
        return HEXLIB_DSP_ERR_NOT_STARTED;
    }

    hexlib_batch_hdr hdr;
    int rc = validate_header(batch, len, rsp_cap, hdr);
    if (rc == HEXLIB_DSP_OK) rc = resolve(ctx, batch, hdr);
    if (rc != HEXLIB_DSP_OK) {
        write_hdr(rsp, (uint32_t) rc, 0, 0);
        return rc;
    }

    ScratchScope scratch_scope(ctx->scratch);
    auto *results = reinterpret_cast<hexlib_op_result *>(rsp + sizeof(hexlib_batch_rsp_hdr));
    uint32_t done = 0;
    uint64_t total_ns = 0;
    int status = HEXLIB_DSP_OK;

    if (use_graph) {
        const bool cached = ctx->graph_exec && ctx->graph_generation == ctx->map_generation &&
                            ctx->graph_blob.size() == len &&
                            std::memcmp(ctx->graph_blob.data(), batch, len) == 0;
        if (!cached) {
            drop_graph(ctx);
            {
                // Validate every op first: a capture must not start on a blob
                // whose op k would refuse.
                DryScope dry_scope(true);
                status = run_ops(ctx, batch, hdr, results, done, false);
            }
            if (status == HEXLIB_DSP_OK && hx::prepare_workspace() != 0) status = HEXLIB_DSP_ERR_INTERNAL;
            if (status == HEXLIB_DSP_OK) {
                StreamScope ss(ctx->stream);
                hexlib_gpu_take_error();
                hipGraph_t graph = nullptr;
                if (hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
                    status = HEXLIB_DSP_ERR_INTERNAL;
                } else {
                    status = run_ops(ctx, batch, hdr, results, done, false);
                    hipError_t ce = hipStreamEndCapture(ctx->stream, &graph);
                    if (ce != hipSuccess || hexlib_gpu_take_error() != 0) status = HEXLIB_DSP_ERR_INTERNAL;
                    if (status == HEXLIB_DSP_OK &&
                        hipGraphInstantiate(&ctx->graph_exec, graph, nullptr, nullptr, 0) != hipSuccess) {
                        ctx->graph_exec = nullptr;
                        status = HEXLIB_DSP_ERR_INTERNAL;
                    }
                    if (graph) hipGraphDestroy(graph);
                }
                if (status == HEXLIB_DSP_OK) {
                    ctx->graph_blob.assign(batch, batch + len);
                    ctx->graph_generation = ctx->map_generation;
                    ctx->graph_nops = hdr.n_ops;
                }
            }
        } else {
            for (uint32_t i = 0; i < hdr.n_ops; ++i) {
                hexlib_op_desc op;
                std::memcpy(&op, batch + hdr.off_ops + (uint64_t) i * sizeof(op), sizeof(op));
                results[i].kind = op.kind;
                results[i].status = HEXLIB_DSP_OK;
                results[i].cycles = 0;
            }
            done = hdr.n_ops;
        }
        if (status == HEXLIB_DSP_OK) {
            if (timed && ensure_events(ctx, 2) != HEXLIB_DSP_OK) status = HEXLIB_DSP_ERR_INTERNAL;
            if (timed) hipEventRecord(ctx->events[0], ctx->stream);
            if (hipGraphLaunch(ctx->graph_exec, ctx->stream) != hipSuccess) status = HEXLIB_DSP_ERR_INTERNAL;
            if (timed) hipEventRecord(ctx->events[1], ctx->stream);
        }
    } else {
        if (timed && ensure_events(ctx, 2 * (size_t) hdr.n_ops) != HEXLIB_DSP_OK) {
            write_hdr(rsp, HEXLIB_DSP_ERR_INTERNAL, 0, 0);
            return HEXLIB_DSP_ERR_INTERNAL;
        }
        DryScope dry_scope(dry);
        StreamScope ss(dry ? (hipStream_t) hexlib_gpu_get_stream() : ctx->stream);
        if (!dry) hexlib_gpu_take_error();
        status = run_ops(ctx, batch, hdr, results, done, timed);
        if (!dry && hexlib_gpu_take_error() != 0 && status == HEXLIB_DSP_OK)
            status = HEXLIB_DSP_ERR_INTERNAL;
    }

    if (!dry && (sync || timed)) {
        if (hipStreamSynchronize(ctx->stream) != hipSuccess && status == HEXLIB_DSP_OK)
            status = HEXLIB_DSP_ERR_INTERNAL;
        if (timed && status == HEXLIB_DSP_OK) {
            float ms = 0.0f;
            if (use_graph) {
                hipEventElapsedTime(&ms, ctx->events[0], ctx->events[1]);
                total_ns = (uint64_t) (ms * 1.0e6);
            } else {
                for (uint32_t i = 0; i < done; ++i) {
                    hipEventElapsedTime(&ms, ctx->events[2 * i], ctx->events[2 * i + 1]);
                    results[i].cycles = (uint64_t) (ms * 1.0e6);
                    total_ns += results[i].cycles;
                }
            }
        }
    }

    write_hdr(rsp, (uint32_t) status, done, total_ns);
    *rsp_len = (uint32_t) (sizeof(hexlib_batch_rsp_hdr) + done * sizeof(hexlib_op_result));
    return status;
}

}  // extern "C"
