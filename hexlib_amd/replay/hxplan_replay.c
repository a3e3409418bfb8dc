/* hxplan_replay: runs a whole-plan file through libhexlib_gpu.so with no
 * Python -- the blob replayed by hexlib_gpu_invoke as a hipGraph.
 *
 *   hxplan_replay PLAN OUTDIR [--reps N] [--input NAME=FILE]...
 *
 * Loads PLAN (arena, const image and stored sample inputs) on device 0,
 * overrides inputs from raw files, runs it once (GRAPH | TIMED) and then N
 * timed replays, writes each graph output to OUTDIR/NAME.bin and prints one
 * JSON line: ops, arena bytes and the mean GPU time of a replay. Exit status
 * 0 on success, else the failing call's status. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "hexlib_gpu.h"

static int fail(const char *what, int rc) {
    fprintf(stderr, "hxplan_replay: %s: %s (%d)\n", what, hexlib_gpu_status_name(rc), rc);
    return rc ? rc : 1;
}

static int run_once(hexlib_gpu_plan *plan, unsigned char *rsp, uint32_t cap, uint64_t *ns) {
    uint32_t len = 0;
    int rc = hexlib_gpu_plan_run(plan, HEXLIB_GPU_INVOKE_GRAPH | HEXLIB_GPU_INVOKE_TIMED, rsp, cap, &len);
    if (rc == HEXLIB_DSP_OK && len >= sizeof(struct hexlib_batch_rsp_hdr)) {
        struct hexlib_batch_rsp_hdr h;
        memcpy(&h, rsp, sizeof(h));
        *ns = h.cycles_total;
    }
    return rc;
}

int main(int argc, char **argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s PLAN OUTDIR [--reps N] [--input NAME=FILE]...\n", argv[0]);
        return 2;
    }
    const char *path = argv[1], *outdir = argv[2];
    int reps = 10;
    hexlib_gpu_ctx *ctx = NULL;
    hexlib_gpu_plan *plan = NULL;
    int rc = hexlib_gpu_open(&ctx);
    if (rc != HEXLIB_DSP_OK) return fail("open", rc);
    rc = hexlib_gpu_start(ctx, 0, 0, 0);
    if (rc != HEXLIB_DSP_OK) return fail("start", rc);
    rc = hexlib_gpu_plan_load(ctx, path, &plan);
    if (rc != HEXLIB_DSP_OK) return fail("plan_load", rc);
    hexlib_plan_info info;
    hexlib_gpu_plan_info_of(plan, &info);

    for (int a = 3; a < argc; ++a) {
        if (!strcmp(argv[a], "--reps") && a + 1 < argc) {
            reps = atoi(argv[++a]);
            continue;
        }
        if (strcmp(argv[a], "--input") || a + 1 >= argc) return fail("arguments", HEXLIB_DSP_ERR_INVAL_PARAMS);
        char *spec = argv[++a], *eq = strchr(spec, '=');
        if (!eq) return fail("--input wants NAME=FILE", HEXLIB_DSP_ERR_INVAL_PARAMS);
        *eq = '\0';
        uint32_t i = 0;
        hexlib_plan_io io;
        for (; i < info.n_io; ++i)
            if (hexlib_gpu_plan_io(plan, i, &io) == HEXLIB_DSP_OK && io.role == 0 && !strcmp(io.name, spec)) break;
        if (i == info.n_io) return fail("no such input", HEXLIB_DSP_ERR_INVAL_PARAMS);
        FILE *f = fopen(eq + 1, "rb");
        void *buf = malloc(io.nbytes ? io.nbytes : 1);
        size_t got = f && buf ? fread(buf, 1, io.nbytes, f) : 0;
        if (f) fclose(f);
        if (got != io.nbytes) return fail("input file size", HEXLIB_DSP_ERR_INVAL_PARAMS);
        rc = hexlib_gpu_plan_write(plan, i, buf, io.nbytes);
        free(buf);
        if (rc != HEXLIB_DSP_OK) return fail("plan_write", rc);
    }

    const uint32_t cap = (uint32_t) (sizeof(struct hexlib_batch_rsp_hdr) +
                                     (info.n_ops + 1) * sizeof(struct hexlib_op_result));
    unsigned char *rsp = (unsigned char *) malloc(cap);
    uint64_t ns = 0, total = 0;
    rc = run_once(plan, rsp, cap, &ns);   /* captures the graph */
    if (rc != HEXLIB_DSP_OK) return fail("first run", rc);
    for (uint32_t i = 0; i < info.n_io; ++i) {
        hexlib_plan_io io;
        hexlib_gpu_plan_io(plan, i, &io);
        if (io.role != 1) continue;
        void *buf = malloc(io.nbytes ? io.nbytes : 1);
        rc = hexlib_gpu_plan_read(plan, i, buf, io.nbytes);
        if (rc != HEXLIB_DSP_OK) return fail("plan_read", rc);
        char name[1024];
        snprintf(name, sizeof(name), "%s/%s.bin", outdir, io.name);
        FILE *f = fopen(name, "wb");
        if (!f || fwrite(buf, 1, io.nbytes, f) != io.nbytes) return fail("output file", HEXLIB_DSP_ERR_INVAL_PARAMS);
        fclose(f);
        free(buf);
    }
    for (int r = 0; r < reps; ++r) {
        rc = run_once(plan, rsp, cap, &ns);
        if (rc != HEXLIB_DSP_OK) return fail("replay", rc);
        total += ns;
    }
    printf("{\"plan\": \"%s\", \"ops\": %u, \"arena_bytes\": %llu, \"reps\": %d, \"gpu_ns_per_run\": %.1f}\n", path,
           info.n_ops, (unsigned long long) info.arena_bytes, reps, reps ? (double) total / reps : 0.0);
    free(rsp);
    rc = hexlib_gpu_plan_free(plan);
    if (rc != HEXLIB_DSP_OK) return fail("plan_free", rc);
    hexlib_gpu_stop(ctx);
    hexlib_gpu_close(ctx);
    return 0;
}
