// The whole-plan file: a plan built once (arena layout, wire blob, const
// image) stored on disk and replayed through hexlib_gpu_invoke with no Python
// on the host. It is the reference's whole-plan batch (hexlib/exec/wholeplan.py:
// 92-357 builds the blob and the arena image; hexlib/tests/test_wholeplan.py:
// 181-183 hands both to the simulator) made into an artefact.
//
// Layout, little-endian, sections back to back:
//   header   64 B   magic "HXPLAN1\0", version 1, the blob's fd, arena bytes,
//                   const bytes, blob bytes, io count, data bytes
//   io table n_io x 96 B: name[48], role (0 input, 1 output), wire dtype id,
//                   arena offset, byte count, ne[4], data offset (inputs that
//                   carry a sample value; UINT64_MAX for none)
//   blob     the wire batch exactly as hexlib/runtime/wire.py:pack_batch writes it
//   const    arena[0, const bytes): weights and other constants, staged
//   data     sample input values
// Loading validates every size and offset on the host first; inspecting a file
// also dry-runs its blob against a mapping of the arena (no HIP call), so a
// malformed file is refused on a machine without a GPU.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "hexlib_gpu.h"

namespace {

constexpr char MAGIC[8] = {'H', 'X', 'P', 'L', 'A', 'N', '1', '\0'};
constexpr uint32_t VERSION = 1;
constexpr uint64_t NO_DATA = ~0ull;

struct FileHeader {
    char magic[8];
    uint32_t version, fd;
    uint64_t arena_bytes, const_bytes, blob_bytes;
    uint32_t n_io, reserved;
    uint64_t data_bytes, reserved2;
};
static_assert(sizeof(FileHeader) == 64, "plan file header is 64 bytes");
static_assert(sizeof(hexlib_plan_io) == 96, "plan file io entry is 96 bytes");

struct Parsed {
    FileHeader h;
    std::vector<hexlib_plan_io> io;
    std::vector<uint8_t> blob, cimg, data;
};

bool read_exact(FILE *f, void *dst, size_t n) { return n == 0 || fread(dst, 1, n, f) == n; }

// Reads and checks the whole file; every offset and size is bounded before use.
int parse(const char *path, Parsed &p) {
    if (!path) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    FILE *f = fopen(path, "rb");
    if (!f) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    int rc = HEXLIB_DSP_OK;
    long size = -1;
    if (fseek(f, 0, SEEK_END) == 0) size = ftell(f);
    rewind(f);
    if (size < (long) sizeof(FileHeader) || !read_exact(f, &p.h, sizeof(FileHeader))) {
        rc = HEXLIB_DSP_ERR_TRUNCATED;
    } else if (memcmp(p.h.magic, MAGIC, sizeof(MAGIC)) != 0) {
        rc = HEXLIB_DSP_ERR_BAD_MAGIC;
    } else if (p.h.version != VERSION) {
        rc = HEXLIB_DSP_ERR_BAD_VERSION;
    } else if (p.h.const_bytes > p.h.arena_bytes || p.h.n_io > 4096 || p.h.blob_bytes > (1ull << 31) ||
               p.h.arena_bytes > (1ull << 40) || p.h.data_bytes > (1ull << 40)) {
        rc = HEXLIB_DSP_ERR_INVAL_PARAMS;
    } else {
        const unsigned __int128 want = (unsigned __int128) sizeof(FileHeader) +
                                       (unsigned __int128) p.h.n_io * sizeof(hexlib_plan_io) + p.h.blob_bytes +
                                       p.h.const_bytes + p.h.data_bytes;
        if (want != (unsigned __int128) size) rc = HEXLIB_DSP_ERR_TRUNCATED;
    }
    if (rc == HEXLIB_DSP_OK) {
        p.io.resize(p.h.n_io);
        p.blob.resize(p.h.blob_bytes);
        p.cimg.resize(p.h.const_bytes);
        p.data.resize(p.h.data_bytes);
        if (!read_exact(f, p.io.data(), p.io.size() * sizeof(hexlib_plan_io)) ||
            !read_exact(f, p.blob.data(), p.blob.size()) || !read_exact(f, p.cimg.data(), p.cimg.size()) ||
            !read_exact(f, p.data.data(), p.data.size()))
            rc = HEXLIB_DSP_ERR_TRUNCATED;
    }
    fclose(f);
    if (rc != HEXLIB_DSP_OK) return rc;
    for (const hexlib_plan_io &e : p.io) {
        if (memchr(e.name, '\0', sizeof(e.name)) == nullptr || e.role > 1) return HEXLIB_DSP_ERR_INVAL_PARAMS;
        if (e.offset > p.h.arena_bytes || e.nbytes > p.h.arena_bytes - e.offset) return HEXLIB_DSP_ERR_INVAL_PARAMS;
        if (e.data_offset != NO_DATA &&
            (e.role != 0 || e.data_offset > p.h.data_bytes || e.nbytes > p.h.data_bytes - e.data_offset))
            return HEXLIB_DSP_ERR_INVAL_PARAMS;
    }
    return HEXLIB_DSP_OK;
}

// Dry-runs the blob against a mapping of the arena: header, tensors, kinds and
// every entry's checks, with no HIP call. Returns the batch status and op count.
int dry_run(const Parsed &p, void *base, uint32_t &n_ops) {
    hexlib_gpu_ctx *ctx = nullptr;
    int rc = hexlib_gpu_open(&ctx);
    if (rc != HEXLIB_DSP_OK) return rc;
    rc = hexlib_gpu_mmap(ctx, p.h.fd, base, p.h.arena_bytes);
    std::vector<uint8_t> rsp(sizeof(hexlib_batch_rsp_hdr) + (size_t) 4096 * sizeof(hexlib_op_result));
    uint32_t len = 0;
    if (rc == HEXLIB_DSP_OK)
        rc = hexlib_gpu_invoke(ctx, p.blob.data(), (uint32_t) p.blob.size(), rsp.data(), (uint32_t) rsp.size(),
                               &len, HEXLIB_GPU_INVOKE_DRYRUN);
    if (len >= sizeof(hexlib_batch_rsp_hdr)) {
        hexlib_batch_rsp_hdr h;
        memcpy(&h, rsp.data(), sizeof(h));
        n_ops = h.n_ops;
    }
    hexlib_gpu_close(ctx);
    return rc;
}

}  // namespace

struct hexlib_gpu_plan {
    hexlib_gpu_ctx *ctx = nullptr;
    Parsed file;
    void *arena = nullptr;
    uint32_t n_ops = 0;
    bool mapped = false;
};

extern "C" {

int hexlib_gpu_plan_inspect(const char *path, hexlib_plan_info *info) {
    Parsed p;
    int rc = parse(path, p);
    if (rc != HEXLIB_DSP_OK) return rc;
    uint32_t n_ops = 0;
    // a host address that is never dereferenced: the dry run only resolves offsets
    rc = dry_run(p, reinterpret_cast<void *>((uintptr_t) 1 << 32), n_ops);
    if (rc != HEXLIB_DSP_OK) return rc;
    if (info) {
        info->version = p.h.version;
        info->fd = p.h.fd;
        info->n_io = p.h.n_io;
        info->n_ops = n_ops;
        info->arena_bytes = p.h.arena_bytes;
        info->const_bytes = p.h.const_bytes;
        info->blob_bytes = p.h.blob_bytes;
        info->data_bytes = p.h.data_bytes;
    }
    return HEXLIB_DSP_OK;
}

int hexlib_gpu_plan_load(hexlib_gpu_ctx *ctx, const char *path, hexlib_gpu_plan **out) {
    if (!ctx || !out) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    *out = nullptr;
    hexlib_gpu_plan *plan = new (std::nothrow) hexlib_gpu_plan();
    if (!plan) return HEXLIB_DSP_ERR_INTERNAL;
    plan->ctx = ctx;
    int rc = parse(path, plan->file);
    const FileHeader &h = plan->file.h;
    if (rc == HEXLIB_DSP_OK) rc = dry_run(plan->file, reinterpret_cast<void *>((uintptr_t) 1 << 32), plan->n_ops);
    if (rc == HEXLIB_DSP_OK && hipMalloc(&plan->arena, h.arena_bytes) != hipSuccess) {
        plan->arena = nullptr;
        rc = HEXLIB_DSP_ERR_MMAP_FAILED;
    }
    if (rc == HEXLIB_DSP_OK && hipMemset(plan->arena, 0, h.arena_bytes) != hipSuccess) rc = HEXLIB_DSP_ERR_INTERNAL;
    if (rc == HEXLIB_DSP_OK && h.const_bytes &&
        hipMemcpy(plan->arena, plan->file.cimg.data(), h.const_bytes, hipMemcpyHostToDevice) != hipSuccess)
        rc = HEXLIB_DSP_ERR_INTERNAL;
    for (size_t i = 0; rc == HEXLIB_DSP_OK && i < plan->file.io.size(); ++i) {
        const hexlib_plan_io &e = plan->file.io[i];
        if (e.data_offset != NO_DATA && e.nbytes &&
            hipMemcpy(static_cast<uint8_t *>(plan->arena) + e.offset, plan->file.data.data() + e.data_offset,
                      e.nbytes, hipMemcpyHostToDevice) != hipSuccess)
            rc = HEXLIB_DSP_ERR_INTERNAL;
    }
    if (rc == HEXLIB_DSP_OK) rc = hexlib_gpu_mmap(ctx, h.fd, plan->arena, h.arena_bytes);
    if (rc == HEXLIB_DSP_OK) {
        plan->mapped = true;
        plan->file.cimg.clear();
        plan->file.cimg.shrink_to_fit();
        *out = plan;
        return HEXLIB_DSP_OK;
    }
    hexlib_gpu_plan_free(plan);
    return rc;
}

int hexlib_gpu_plan_info_of(const hexlib_gpu_plan *plan, hexlib_plan_info *info) {
    if (!plan || !info) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    const FileHeader &h = plan->file.h;
    info->version = h.version;
    info->fd = h.fd;
    info->n_io = h.n_io;
    info->n_ops = plan->n_ops;
    info->arena_bytes = h.arena_bytes;
    info->const_bytes = h.const_bytes;
    info->blob_bytes = h.blob_bytes;
    info->data_bytes = h.data_bytes;
    return HEXLIB_DSP_OK;
}

int hexlib_gpu_plan_io(const hexlib_gpu_plan *plan, uint32_t i, hexlib_plan_io *io) {
    if (!plan || !io || i >= plan->file.io.size()) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    *io = plan->file.io[i];
    return HEXLIB_DSP_OK;
}

int hexlib_gpu_plan_write(hexlib_gpu_plan *plan, uint32_t i, const void *host, uint64_t nbytes) {
    if (!plan || !host || i >= plan->file.io.size()) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    const hexlib_plan_io &e = plan->file.io[i];
    if (e.role != 0 || nbytes != e.nbytes) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    return hipMemcpy(static_cast<uint8_t *>(plan->arena) + e.offset, host, nbytes, hipMemcpyHostToDevice) ==
                   hipSuccess
               ? HEXLIB_DSP_OK
               : HEXLIB_DSP_ERR_INTERNAL;
}

int hexlib_gpu_plan_read(const hexlib_gpu_plan *plan, uint32_t i, void *host, uint64_t nbytes) {
    if (!plan || !host || i >= plan->file.io.size()) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    const hexlib_plan_io &e = plan->file.io[i];
    if (nbytes != e.nbytes) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    return hipMemcpy(host, static_cast<const uint8_t *>(plan->arena) + e.offset, nbytes, hipMemcpyDeviceToHost) ==
                   hipSuccess
               ? HEXLIB_DSP_OK
               : HEXLIB_DSP_ERR_INTERNAL;
}

int hexlib_gpu_plan_run(hexlib_gpu_plan *plan, uint32_t flags, uint8_t *rsp, uint32_t rsp_cap, uint32_t *rsp_len) {
    if (!plan) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    return hexlib_gpu_invoke(plan->ctx, plan->file.blob.data(), (uint32_t) plan->file.blob.size(), rsp, rsp_cap,
                             rsp_len, flags);
}

int hexlib_gpu_plan_free(hexlib_gpu_plan *plan) {
    if (!plan) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    int rc = HEXLIB_DSP_OK;
    if (plan->mapped) rc = hexlib_gpu_munmap(plan->ctx, plan->file.h.fd);
    if (plan->arena && hipFree(plan->arena) != hipSuccess) rc = HEXLIB_DSP_ERR_INTERNAL;
    delete plan;
    return rc;
}

}  // extern "C"
