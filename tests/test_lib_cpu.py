"""The C-ABI library on the CPU: it loads, exports every declared symbol, its
wire structs match the Python serializer byte for byte, the generated entries
are current, and every refusal of the dispatcher fires before any GPU call.

No compute runs here: DRYRUN invokes validate the blob, resolve tensors and
run the generated entries' checks, and the API functions return before
launching (the library makes no HIP call on that path). The refusals restate
the reference's host-forced failures (`hexlib/exec/dsp.py:565-609`,
`hexlib/tests/test_dsp_sim.py:43-706`): bad magic, bad version, truncation,
an unmapped buffer, an unknown kind, a dtype or layout mismatch.
"""
import ctypes
import struct

import numpy as np
import pytest

from hexlib_amd import lib as L
from hexlib_amd.exec import genentry, wire
from hexlib_amd.exec.runner import KIND_ID, SPECS

OK = wire.STATUS["OK"]


@pytest.fixture(scope="module")
def lib():
    return L.load()


def test_every_declared_symbol_is_exported(lib):
    names = L.header_functions() + L.header_objects()
    assert len(names) > 40
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/hexlib_gpu.h but not exported"


def test_struct_sizes_match_the_wire(lib):
    arr = (ctypes.c_uint32 * 8)()
    n = lib.hexlib_gpu_struct_sizes(arr, 8)
    assert list(arr)[:6] == [wire.HDR_SIZE, wire.BUF_SIZE, wire.TENSOR_SIZE, wire.OP_SIZE,
                             wire.RSP_HDR_SIZE, wire.RESULT_SIZE]
    assert n == 7


def test_status_names_agree(lib):
    for name, code in wire.STATUS.items():
        assert lib.hexlib_gpu_status_name(code).decode() == name


def test_generated_entries_are_current():
    assert open(genentry.OUT_PATH).read() == genentry.generate()


def test_kernel_table_covers_every_spec(lib):
    n = ctypes.c_uint32.in_dll(lib, "hexlib_kernel_table_len").value
    assert n == len(SPECS)


# ---- dispatcher refusals, all on the host -------------------------------------

class Session:
    def __init__(self, lib):
        self.lib = lib
        self.h = ctypes.c_void_p()
        assert lib.hexlib_gpu_open(ctypes.byref(self.h)) == OK

    def mmap(self, fd, size, base=0x10000000):
        return self.lib.hexlib_gpu_mmap(self.h, fd, ctypes.c_void_p(base), size)

    def invoke(self, blob, flags=L.INVOKE_DRYRUN, cap=4096):
        rsp = ctypes.create_string_buffer(cap)
        n = ctypes.c_uint32()
        rc = self.lib.hexlib_gpu_invoke(self.h, blob, len(blob), rsp, cap, ctypes.byref(n), flags)
        return rc, wire.unpack_response(rsp.raw[:n.value])

    def close(self):
        self.lib.hexlib_gpu_close(self.h)


@pytest.fixture
def sess(lib):
    s = Session(lib)
    yield s
    s.close()


def scale_blob(fd=3, n=4100, dtype_in="fp16", layout="row_major", kind=None, out_n=None,
               size=None):
    nb = n * (4 if dtype_in == "fp32" else 2)
    out_n = n if out_n is None else out_n
    off_out = (nb + 255) // 256 * 256
    size = size or off_out + out_n * 2
    t = [wire.TensorDesc(0, 0, nb, dtype_in, layout, (n, 1, 1, 1)),
         wire.TensorDesc(0, off_out, out_n * 2, "fp16", "row_major", (out_n, 1, 1, 1))]
    op = wire.OpDesc(kind if kind is not None else KIND_ID["scale"],
                     (wire.float_param(0.125),), (0,), (1,))
    return wire.pack_batch([wire.BufDesc(fd, size)], t, [op]), size


def test_dry_run_accepts_a_well_formed_op(sess):
    blob, size = scale_blob()
    assert sess.mmap(3, size) == OK
    rc, rsp = sess.invoke(blob)
    assert rc == OK and rsp.ok and rsp.arch == 950
    assert [r.kind for r in rsp.results] == [KIND_ID["scale"]]


def test_invoke_before_start_is_refused(sess):
    blob, size = scale_blob()
    sess.mmap(3, size)
    rc, rsp = sess.invoke(blob, flags=0)
    assert rc == rsp.status == wire.STATUS["ERR_NOT_STARTED"]


def test_bad_magic_and_version(sess):
    blob, size = scale_blob()
    sess.mmap(3, size)
    bad = bytearray(blob)
    bad[0] ^= 1
    assert sess.invoke(bytes(bad))[0] == wire.STATUS["ERR_BAD_MAGIC"]
    bad = bytearray(blob)
    struct.pack_into("<I", bad, 4, 2)
    assert sess.invoke(bytes(bad))[0] == wire.STATUS["ERR_BAD_VERSION"]


def test_truncated_blob_and_response(sess):
    blob, size = scale_blob()
    sess.mmap(3, size)
    assert sess.invoke(blob[:-4])[0] == wire.STATUS["ERR_TRUNCATED"]
    assert sess.invoke(blob[:10])[0] == wire.STATUS["ERR_TRUNCATED"]
    assert sess.invoke(blob, cap=wire.RSP_HDR_SIZE)[0] == wire.STATUS["ERR_TRUNCATED"]


def test_huge_op_count_cannot_wrap_the_bounds_check(sess):
    blob, size = scale_blob()
    sess.mmap(3, size)
    bad = bytearray(blob)
    struct.pack_into("<I", bad, 20, 0xFFFFFFFF)
    assert sess.invoke(bytes(bad))[0] == wire.STATUS["ERR_TRUNCATED"]


def test_an_unmapped_fd_is_refused(sess):
    blob, size = scale_blob(fd=9)
    sess.mmap(3, size)
    assert sess.invoke(blob)[0] == wire.STATUS["ERR_UNMAPPED"]


def test_buffer_larger_than_its_mapping_is_refused(sess):
    blob, size = scale_blob()
    sess.mmap(3, size - 256)
    assert sess.invoke(blob)[0] == wire.STATUS["ERR_INVAL_PARAMS"]


def test_unknown_kind_is_no_kernel(sess):
    blob, size = scale_blob(kind=99)
    sess.mmap(3, size)
    rc, rsp = sess.invoke(blob)
    assert rc == wire.STATUS["ERR_NO_KERNEL"] and rsp.results[0].kind == 99


def test_reshape_kind_has_no_kernel(sess):
    blob, size = scale_blob(kind=KIND_ID["reshape"])
    sess.mmap(3, size)
    assert sess.invoke(blob)[0] == wire.STATUS["ERR_NO_KERNEL"]


def test_dtype_and_layout_mismatch_are_requires(sess):
    blob, size = scale_blob(dtype_in="fp32", n=2050)
    sess.mmap(3, size)
    assert sess.invoke(blob)[0] == wire.STATUS["ERR_REQUIRES"]
    blob, size = scale_blob(fd=4, layout="tiled_32x32")
    sess.mmap(4, size, base=0x30000000)
    assert sess.invoke(blob)[0] == wire.STATUS["ERR_REQUIRES"]


def test_output_smaller_than_the_kernel_writes_is_refused(sess):
    blob, size = scale_blob(out_n=100)
    sess.mmap(3, size)
    assert sess.invoke(blob)[0] == wire.STATUS["ERR_INVAL_PARAMS"]


def test_extent_larger_than_nbytes_is_refused(sess):
    n = 4100
    t = [wire.TensorDesc(0, 0, 100, "fp16", "row_major", (n, 1, 1, 1)),
         wire.TensorDesc(0, 8448, n * 2, "fp16", "row_major", (n, 1, 1, 1))]
    op = wire.OpDesc(KIND_ID["scale"], (wire.float_param(0.5),), (0,), (1,))
    blob = wire.pack_batch([wire.BufDesc(3, 8448 + n * 2)], t, [op])
    sess.mmap(3, 8448 + n * 2)
    assert sess.invoke(blob)[0] == wire.STATUS["ERR_INVAL_PARAMS"]


@pytest.mark.parametrize("ne,want", [
    ((2, 4, 8, 1), "OK"),                                  # 64 elements in 128 bytes
    ((2, 8, 8, 1), "ERR_INVAL_PARAMS"),                    # an honest oversize
    ((1 << 15, 1 << 19, 1 << 30, 1), "ERR_INVAL_PARAMS"),  # B*T*D = 2^64: wraps to 0 in 64 bits
    ((1 << 16, 1 << 16, 1 << 16, 1 << 16), "ERR_INVAL_PARAMS"),  # numel 2^64 with a fourth axis
    # 64 * (2^29 + 2^15 + 1) * (2^29 - 2^15 + 1) = 2^64 + 64: wraps to exactly 64
    ((64, (1 << 29) + (1 << 15) + 1, (1 << 29) - (1 << 15) + 1, 1), "ERR_INVAL_PARAMS"),
])
def test_extents_that_wrap_64_bits_are_refused(sess, ne, want):
    """Both sides of every capacity check (the extent the kernel will touch
    and the buffer's element count, and the element count against nbytes) are
    computed without wrapping: a crafted ne whose products wrap to a small
    value in 64-bit arithmetic must not pass as a 64-element tensor."""
    t = [wire.TensorDesc(0, 0, 128, "fp16", "row_major", ne),
         wire.TensorDesc(0, 256, 128, "fp16", "row_major", (ne[0], ne[2], ne[1], ne[3]))]
    op = wire.OpDesc(KIND_ID["transpose_hd"], (), (0,), (1,))
    blob = wire.pack_batch([wire.BufDesc(3, 512)], t, [op])
    sess.mmap(3, 512)
    assert sess.invoke(blob)[0] == wire.STATUS[want]


def test_patchify_extent_with_seven_factors_saturates(sess):
    """patchify's output extent multiplies seven checked ints; a product past
    2^128 saturates instead of wrapping."""
    big = 0x7fffffff
    t = [wire.TensorDesc(0, 0, 256, "fp32", "row_major", (3, 1, 4, 4)),
         wire.TensorDesc(0, 256, 256, "fp32", "row_major", (64, 1, 1, 1))]
    op = wire.OpDesc(KIND_ID["patchify"], (big, big, big, big, 1), (0,), (1,))
    blob = wire.pack_batch([wire.BufDesc(3, 512)], t, [op])
    sess.mmap(3, 512)
    assert sess.invoke(blob)[0] == wire.STATUS["ERR_INVAL_PARAMS"]


def test_bad_activation_code_is_refused(sess):
    M, K, N = 4, 64, 32
    sizes = [M * K * 2, K * N // 32 * 18, N * 4, M * N * 2]
    offs = np.cumsum([0] + [(s + 255) // 256 * 256 for s in sizes])
    t = [wire.TensorDesc(0, int(offs[0]), sizes[0], "fp16", "row_major", (M, K, 1, 1)),
         wire.TensorDesc(0, int(offs[1]), sizes[1], "q4_0", "row_major", (K, N, 1, 1)),
         wire.TensorDesc(0, int(offs[2]), sizes[2], "fp32", "row_major", (N, 1, 1, 1)),
         wire.TensorDesc(0, int(offs[3]), sizes[3], "fp16", "row_major", (M, N, 1, 1))]
    for act, want in ((1, "OK"), (7, "ERR_INVAL_PARAMS")):
        op = wire.OpDesc(KIND_ID["matmul_epilogue"], (act,), (0, 1, 2), (3,))
        blob = wire.pack_batch([wire.BufDesc(3, int(offs[4]))], t, [op])
        sess.mmap(3, int(offs[4]))
        assert sess.invoke(blob)[0] == wire.STATUS[want]


def test_first_failing_op_stops_the_batch(sess):
    blob, size = scale_blob()
    hdr = list(struct.unpack_from(wire._HDR, blob))
    n_ops = 3
    ops = blob[hdr[8]:] * 1
    good = ops
    bad = bytearray(ops)
    struct.pack_into("<I", bad, 0, 99)
    body = blob[:hdr[8]] + good + bytes(bad) + good
    body = bytearray(body)
    struct.pack_into("<I", body, 8, len(body))
    struct.pack_into("<I", body, 20, n_ops)
    sess.mmap(3, size)
    rc, rsp = sess.invoke(bytes(body))
    assert rc == wire.STATUS["ERR_NO_KERNEL"]
    assert rsp.n_ops == 2 and rsp.results[0].ok and rsp.results[1].status == rc


def test_mmap_table_limits(sess):
    for fd in range(32):
        assert sess.mmap(100 + fd, 256, 0x20000000 + fd * 4096) == OK
    assert sess.mmap(500, 256, 0x90000000) == wire.STATUS["ERR_NO_MMAP_SLOT"]
    assert sess.mmap(100, 256, 0x20000000) == OK                        # idempotent
    assert sess.mmap(100, 512, 0x20000000) == wire.STATUS["ERR_MMAP_FAILED"]
    assert sess.lib.hexlib_gpu_munmap(sess.h, 100) == OK
    assert sess.lib.hexlib_gpu_munmap(sess.h, 100) == wire.STATUS["ERR_UNMAPPED"]


def test_whole_encoder_blob_dry_runs(sess):
    from hexlib_amd import encoder as E
    from hexlib_amd.exec.wholeplan import build_whole_plan_batch
    cfg = E.TINY_ENCODER
    g = E.build_vision_encoder(cfg)
    wb = build_whole_plan_batch(g, E.synthetic_feeds(g, cfg))
    sess.mmap(0, wb.arena_bytes)
    rc, rsp = sess.invoke(wb.blob, cap=wire.RSP_HDR_SIZE + wire.RESULT_SIZE * wb.n_ops)
    assert rc == OK and rsp.n_ops == wb.n_ops and rsp.ok


def _attention_blob(rows, H, D, batch, align_out=0):
    n = rows * H * D * 2
    step = (n + 255) // 256 * 256
    t = [wire.TensorDesc(0, i * step, n, "fp16", "row_major", (rows, H, D, 1)) for i in range(3)]
    t.append(wire.TensorDesc(0, 3 * step + align_out, n, "fp16", "row_major", (rows, H, D, 1)))
    op = wire.OpDesc(KIND_ID["attention"], (batch, wire.float_param(D ** -0.5)), (0, 1, 2), (3,))
    return wire.pack_batch([wire.BufDesc(3, 4 * step + 256)], t, [op]), 4 * step + 256


@pytest.mark.parametrize("rows,H,D,batch,align_out,want", [
    (256, 12, 64, 1, 0, "OK"), (66, 2, 32, 2, 0, "OK"),
    (256, 12, 48, 1, 0, "ERR_INVAL_PARAMS"),      # head_dim the kernel has no tile for
    (257, 2, 64, 2, 0, "ERR_INVAL_PARAMS"),       # rows do not split into images
    (64, 2, 64, 0, 0, "ERR_INVAL_PARAMS"),        # batch 0
    (64, 2, 64, 1, 2, "ERR_INVAL_PARAMS"),        # misaligned output
    (64, 2, 64, 1, 8, "ERR_INVAL_PARAMS")])
def test_attention_entry_checks(sess, rows, H, D, batch, align_out, want):
    blob, size = _attention_blob(rows, H, D, batch, align_out)
    assert sess.mmap(3, size) == OK
    assert sess.invoke(blob)[0] == wire.STATUS[want]


@pytest.mark.parametrize("two,three,D,want", [(2, 3, 64, "OK"), (3, 3, 64, "ERR_INVAL_PARAMS"),
                                              (2, 2, 64, "ERR_INVAL_PARAMS"), (2, 3, 40, "ERR_INVAL_PARAMS")])
def test_attention_qk_v_entry_checks(sess, two, three, D, want):
    rows, H = 64, 2
    sizes = [rows * two * H * D * 2, rows * three * H * D * 2, rows * H * D * 2]
    offs = np.cumsum([0] + [(x + 255) // 256 * 256 for x in sizes])
    t = [wire.TensorDesc(0, int(offs[0]), sizes[0], "fp16", "row_major", (rows, two, H, D)),
         wire.TensorDesc(0, int(offs[1]), sizes[1], "fp16", "row_major", (rows, three, H, D)),
         wire.TensorDesc(0, int(offs[2]), sizes[2], "fp16", "row_major", (rows, H, D, 1))]
    op = wire.OpDesc(KIND_ID["attention_qk_v"], (1, wire.float_param(0.125)), (0, 1), (2,))
    blob = wire.pack_batch([wire.BufDesc(3, int(offs[3]))], t, [op])
    assert sess.mmap(3, int(offs[3])) == OK
    assert sess.invoke(blob)[0] == wire.STATUS[want]


def _blob(kind, tensors, params, n_src):
    """One op over tensors laid out back to back at 256-byte steps."""
    offs, descs, cur = [], [], 0
    for shape, dt, lay in tensors:
        n = int(np.prod(shape)) * (2 if dt == "fp16" else 4)
        descs.append(wire.TensorDesc(0, cur, n, dt, lay, wire.pad_ne(shape)))
        cur += (n + 255) // 256 * 256
    op = wire.OpDesc(KIND_ID[kind], params, tuple(range(n_src)), (n_src,))
    return wire.pack_batch([wire.BufDesc(3, cur)], descs, [op]), cur


@pytest.mark.parametrize("M,K,N,heads,d,table_layout,want", [
    (256, 768, 2304, 12, 64, "col_major", "OK"), (65, 128, 192, 2, 32, "col_major", "OK"),
    (64, 64, 128, 2, 32, "col_major", "OK"),
    (64, 96, 192, 2, 32, "col_major", "ERR_INVAL_PARAMS"),    # K not a multiple of 64
    (64, 128, 192, 2, 30, "col_major", "ERR_INVAL_PARAMS"),   # rope_dim not a multiple of 4
    (64, 128, 192, 4, 32, "col_major", "ERR_INVAL_PARAMS"),   # 2 * heads * rope_dim > N
    (64, 128, 192, 2, 32, "row_major", "ERR_REQUIRES")])      # tables not stored transposed
def test_matmul_epilogue_rope_entry_checks(sess, M, K, N, heads, d, table_layout, want):
    blob, size = _blob("matmul_epilogue_f16wt_rope",
                       [((M, K), "fp16", "row_major"), ((K, N), "fp16", "col_major_rope"),
                        ((N,), "fp32", "row_major"), ((M, d), "fp32", table_layout),
                        ((M, d), "fp32", "col_major"), ((M, N), "fp16", "row_major")],
                       (0, heads, d), 5)
    assert sess.mmap(3, size) == OK
    assert sess.invoke(blob)[0] == wire.STATUS[want]


@pytest.mark.parametrize("three,D,batch,want", [(3, 64, 1, "OK"), (3, 32, 2, "OK"), (2, 64, 1, "ERR_INVAL_PARAMS"),
                                                (3, 48, 1, "ERR_INVAL_PARAMS"), (3, 64, 3, "ERR_INVAL_PARAMS")])
def test_attention_qkv_entry_checks(sess, three, D, batch, want):
    rows, H = 64, 2
    blob, size = _blob("attention_qkv", [((rows, three, H, D), "fp16", "row_major"),
                                         ((rows, H, D), "fp16", "row_major")],
                       (batch, wire.float_param(D ** -0.5)), 1)
    assert sess.mmap(3, size) == OK
    assert sess.invoke(blob)[0] == wire.STATUS[want]


def test_col_major_rope_staging_matches_the_oracle_permutation():
    """The product's staging of a col_major_rope weight against the oracle's
    row-by-row restatement; rows past the 2 * heads rope heads (the v slot)
    stay plain W^T, and the permutation is a bijection on each head."""
    from hexlib_amd.exec.wholeplan import stage_col_major_rope
    from oracle import kernels as K
    r = np.random.default_rng(2)
    for Kd, heads, d, N in ((64, 2, 32, 192), (128, 3, 8, 80), (64, 12, 64, 2304)):
        w = r.standard_normal((Kd, N)).astype(np.float16)
        got = np.frombuffer(stage_col_major_rope(w, heads, d), np.float16).reshape(N, Kd)
        want = K.permute_rope_rows(w.T, heads, d)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(got[2 * heads * d:], w.T[2 * heads * d:])
        for h in range(2 * heads):
            blk = got[h * d:(h + 1) * d]
            np.testing.assert_array_equal(blk[0::2], w.T[h * d:h * d + d // 2])
            np.testing.assert_array_equal(blk[1::2], w.T[h * d + d // 2:(h + 1) * d])


@pytest.mark.parametrize("M,K,N,want", [(256, 768, 3072, "OK"), (65, 512, 200, "OK"), (64, 640, 64, "OK"),
                                        (64, 448, 64, "ERR_INVAL_PARAMS"),     # row block below 512
                                        (64, 832, 64, "ERR_INVAL_PARAMS"),     # row block past 768
                                        (64, 600, 64, "ERR_INVAL_PARAMS")])    # K not a multiple of 64
def test_layernorm_matmul_entry_checks(sess, M, K, N, want):
    blob, size = _blob("layernorm_matmul_epilogue_f16wt",
                       [((M, K), "fp16", "row_major"), ((K,), "fp32", "row_major"), ((K,), "fp32", "row_major"),
                        ((K, N), "fp16", "col_major"), ((N,), "fp32", "row_major"), ((M, N), "fp16", "row_major")],
                       (1, wire.float_param(1e-6)), 5)
    assert sess.mmap(3, size) == OK
    assert sess.invoke(blob)[0] == wire.STATUS[want]


@pytest.mark.parametrize("K,layout,want", [(768, "q8_0_kgroup", "OK"), (96, "q8_0_kgroup", "OK"),
                                           (768, "q4_0_kgroup", "ERR_REQUIRES")])
def test_matmul_q8k_entry_checks(sess, K, layout, want):
    M, N = 16, 64
    blob, size = _blob("matmul_epilogue_q8k",
                       [((M, K), "fp16", "row_major"), ((K, N), "q8_0", layout),
                        ((N,), "fp32", "row_major"), ((M, N), "fp16", "row_major")], (0,), 3)
    assert sess.mmap(3, size) == OK
    assert sess.invoke(blob)[0] == wire.STATUS[want]
