"""Helpers for GPU tests: device buffers from numpy, C-ABI calls on torch's
stream, loud failure on any launch error."""
import ctypes

import numpy as np

from hexlib_amd import lib as L


class Dev:
    def __init__(self, torch):
        self.torch = torch
        self.lib = L.load()
        self.lib.hexlib_gpu_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        self.lib.hexlib_gpu_take_error()

    def up(self, arr, offset_bytes: int = 0):
        """Copy a numpy array to the device. A nonzero `offset_bytes` returns a
        view that starts that many bytes into a fresh buffer (misaligned base)."""
        a = np.ascontiguousarray(arr)
        raw = a.view(np.uint8).reshape(-1)
        buf = self.torch.zeros(raw.size + offset_bytes + 256, dtype=self.torch.uint8, device="cuda")
        buf[offset_bytes:offset_bytes + raw.size].copy_(self.torch.from_numpy(raw.copy()))
        return (buf, offset_bytes, a.dtype, a.shape)

    def empty(self, shape, dtype, offset_bytes: int = 0, fill: float = 12345.0):
        """Output buffer pre-filled with a poison value (the reference harnesses
        poison outputs with 12345.0 so an unwritten element cannot pass)."""
        a = np.full(shape, fill, dtype=dtype)
        return self.up(a, offset_bytes)

    def ptr(self, d):
        buf, off, _, _ = d
        return ctypes.c_void_p(buf.data_ptr() + off)

    def down(self, d):
        self.torch.cuda.synchronize()
        buf, off, dtype, shape = d
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        raw = buf[off:off + n].cpu().numpy()
        return raw.view(dtype).reshape(shape).copy()

    def check(self):
        self.torch.cuda.synchronize()
        err = self.lib.hexlib_gpu_take_error()
        assert err == 0, f"HIP launch error: {self.lib.hexlib_gpu_error_string(err).decode()}"


def h16(a):
    return np.asarray(a, dtype=np.float16)


def report(name, got, want):
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    d = np.abs(g - w)
    print(f"[{name}] max abs {d.max():.3e}  max rel {(d / np.maximum(np.abs(w), 1e-6)).max():.3e}",
          flush=True)
    return d.max()
