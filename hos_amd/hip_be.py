"""Python mirror of the reference's GPU boundary (the Rust `Gpu` method set, src/metal_be_stub.rs:35-208)
over the C ABI of libhos_hip.so.

Method names, argument order and meaning follow the Rust surface: ``matmul_f32_keyed(a, m, k, b, n, b_key)``
returns ``C = A·B``; ``matmul_abt_keyed(a, m, n, b, k, b_key)`` returns ``A·Bᵀ``; ``matmul_atb_keyed(a, k, m, b,
n, a_key)`` returns ``Aᵀ·B``; ``b_key=None`` means "no caching". Where the reference panics, this raises
``HosError`` carrying the C status code.
"""
import ctypes
import weakref

import numpy as np

from ._lib import lib

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q5_0, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_BF16 = \
    0, 1, 2, 6, 8, 12, 13, 14, 30
# elements per block of each weight encoding upload_quant takes (src/gguf.rs:330-505)
BLOCK = {GGML_F32: 1, GGML_F16: 1, GGML_BF16: 1, GGML_Q4_0: 32, GGML_Q5_0: 32, GGML_Q8_0: 32, GGML_Q4_K: 256,
         GGML_Q5_K: 256, GGML_Q6_K: 256}

STATUS = {1: "Io", 2: "Format", 3: "MissingTensor", 4: "UnsupportedQuant", 5: "UnsupportedArch",
          6: "MissingMeta", 7: "Spec", 8: "Device", 9: "Invalid", 10: "OutOfMemory"}


class HosError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{STATUS.get(code, code)}] {msg}")
        self.code = code


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def bytes_for(ggml_type, n):
    """bytes_for (src/gguf.rs:548-561); 0 for unsupported types."""
    return lib().hos_hip_bytes_for(ggml_type, n)


class Gpu:
    """One device context (Gpu::new). Not thread-safe, like the reference's thread-local Gpu."""

    def __init__(self, device=0):
        h = ctypes.c_void_p()
        rc = lib().hos_hip_create(device, ctypes.byref(h))
        if rc:
            raise HosError(rc, f"hos_hip_create(device={device}) failed (no usable HIP device?)")
        self.h = h
        self._children = weakref.WeakSet()  # objects that live on this context; closed before it

    def adopt(self, obj):
        self._children.add(obj)

    def close(self):
        if getattr(self, "h", None):
            for c in list(getattr(self, "_children", ())):
                c.close()
            lib().hos_hip_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _chk(self, rc):
        if rc:
            raise HosError(rc, lib().hos_hip_last_error(self.h).decode())

    def arch(self):
        buf = ctypes.create_string_buffer(64)
        self._chk(lib().hos_hip_device_arch(self.h, buf, 64))
        return buf.value.decode()

    def synchronize(self):
        self._chk(lib().hos_hip_synchronize(self.h))

    def set_gemm_passes(self, passes):
        """qGEMM precision: 1 fp16 pass, 2 (activation hi+lo), 3 (activation and weight hi+lo)."""
        self._chk(lib().hos_hip_set_gemm_passes(self.h, passes))

    # ---- keyed f32 GEMMs (src/metal_be.rs:2338-2366, 2434-2446) ----
    def matmul_f32_keyed(self, a, m, k, b, n, b_key=None):
        a, b = _f32(a), _f32(b)
        out = np.empty((m, n), np.float32)
        self._chk(lib().hos_hip_matmul_f32_keyed(self.h, _p(a), m, k, _p(b), n, b_key or 0, _p(out)))
        return out

    def matmul_abt_keyed(self, a, m, n, b, k, b_key=None):
        a, b = _f32(a), _f32(b)
        out = np.empty((m, k), np.float32)
        self._chk(lib().hos_hip_matmul_abt_keyed(self.h, _p(a), m, n, _p(b), k, b_key or 0, _p(out)))
        return out

    def matmul_atb_keyed(self, a, k, m, b, n, a_key=None):
        a, b = _f32(a), _f32(b)
        out = np.empty((k, n), np.float32)
        self._chk(lib().hos_hip_matmul_atb_keyed(self.h, _p(a), k, m, _p(b), n, a_key or 0, _p(out)))
        return out

    def evict(self, key):
        self._chk(lib().hos_hip_evict(self.h, key))

    def clear_cache(self):
        self._chk(lib().hos_hip_clear_cache(self.h))

    # ---- quantized frozen weights ----
    def upload_quant(self, key, raw, ggml_type, rows, cols):
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        self._chk(lib().hos_hip_upload_quant(self.h, key, _p(raw), raw.size, ggml_type, rows, cols))
        return (key, ggml_type, rows, cols)

    def dequant(self, key, rows, cols):
        out = np.empty((rows, cols), np.float32)
        self._chk(lib().hos_hip_dequant(self.h, key, _p(out)))
        return out

    def qgemm_fwd(self, key, x, rows):
        """Y = X·deq(W)ᵀ for an uploaded W [rows, cols]; x: [t, cols]."""
        x = _f32(x)
        out = np.empty((x.shape[0], rows), np.float32)
        self._chk(lib().hos_hip_qgemm_fwd(self.h, key, _p(x), x.shape[0], _p(out)))
        return out

    def qgemm_dx(self, key, dy, cols):
        """dX = dY·deq(W) for an uploaded W [rows, cols]; dy: [t, rows]."""
        dy = _f32(dy)
        out = np.empty((dy.shape[0], cols), np.float32)
        self._chk(lib().hos_hip_qgemm_dx(self.h, key, _p(dy), dy.shape[0], _p(out)))
        return out

    def quantize(self, x, ggml_type):
        """quantize(x, type) of src/gguf_write.rs:41-50, on the device."""
        x = _f32(x).ravel()
        out = np.empty(bytes_for(ggml_type, x.size), np.uint8)
        self._chk(lib().hos_hip_quantize(self.h, _p(x), x.size, ggml_type, _p(out)))
        return out

    def random_quantized(self, rows, cols, ggml_type, seed, stddev=0.02):
        """Quantized bytes of a [rows, cols] ~N(0, stddev²) matrix drawn and quantized on the device (fast
        synthetic weights for very large tensors), in chunks of whole rows."""
        out = np.empty(bytes_for(ggml_type, rows * cols), np.uint8)
        chunk = max(1, (64 << 20) // cols)
        x, q = self.alloc(chunk * cols * 4), self.alloc(bytes_for(ggml_type, chunk * cols))
        try:
            done = 0
            for r0 in range(0, rows, chunk):
                n = min(chunk, rows - r0) * cols
                self._chk(lib().hos_hip_randn_dev(self.h, x, n, (seed << 20) + r0 // chunk, stddev))
                self._chk(lib().hos_hip_quantize_dev(self.h, x, n, ggml_type, q))
                nb = bytes_for(ggml_type, n)
                self._chk(lib().hos_hip_d2h(self.h, _p(out[done:done + nb]), q, nb))
                done += nb
        finally:
            self.free(x)
            self.free(q)
        return out

    # ---- device memory ----
    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        self._chk(lib().hos_hip_dev_alloc(self.h, nbytes, ctypes.byref(p)))
        return p

    def free(self, p):
        self._chk(lib().hos_hip_dev_free(self.h, p))

    def h2d(self, dst, arr):
        arr = np.ascontiguousarray(arr)
        self._chk(lib().hos_hip_h2d(self.h, dst, _p(arr), arr.nbytes))

    def d2h(self, src, shape, dtype):
        out = np.empty(shape, dtype)
        self._chk(lib().hos_hip_d2h(self.h, _p(out), src, out.nbytes))
        return out

    def time_qgemm(self, which, key, in_dev, t, out_dev, iters):
        ms = ctypes.c_float()
        self._chk(lib().hos_hip_time_qgemm(self.h, which, key, in_dev, t, out_dev, iters, ctypes.byref(ms)))
        return ms.value

    def timer_begin(self):
        """Start timing the context stream (HIP event); pair with timer_end."""
        self._chk(lib().hos_hip_timer_begin(self.h))

    def timer_end(self):
        """Milliseconds of stream work since timer_begin (waits for the stream)."""
        ms = ctypes.c_float()
        self._chk(lib().hos_hip_timer_end(self.h, ctypes.byref(ms)))
        return ms.value

    def op_async(self, name, *args):
        """Enqueue hos_hip_<name>(ctx, *args) without waiting for the stream."""
        conv = [a.ptr if isinstance(a, DevArray) else a for a in args]
        self._chk(getattr(lib(), "hos_hip_" + name)(self.h, *conv))

    # ---- op-level entry points (device pointers) ----
    def to_dev(self, arr):
        """Upload an array; returns a DevArray that frees itself with .free()."""
        arr = np.ascontiguousarray(arr)
        d = DevArray(self, arr.shape, arr.dtype)
        self.h2d(d.ptr, arr)
        return d

    def empty_dev(self, shape, dtype=np.float32, fill=None):
        d = DevArray(self, shape, dtype)
        if fill is not None:
            self.h2d(d.ptr, np.full(shape, fill, dtype))
        return d

    def op(self, name, *args):
        """Call hos_hip_<name>(ctx, *args) (DevArray arguments pass their pointers), then synchronize."""
        conv = [a.ptr if isinstance(a, DevArray) else a for a in args]
        self._chk(getattr(lib(), "hos_hip_" + name)(self.h, *conv))
        self.synchronize()


class DevArray:
    """A device allocation of a given shape/dtype owned through a Gpu context."""

    def __init__(self, gpu, shape, dtype):
        self.gpu, self.shape, self.dtype = gpu, tuple(shape), np.dtype(dtype)
        nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = gpu.alloc(max(nbytes, 4))

    def get(self):
        return self.gpu.d2h(self.ptr, self.shape, self.dtype)

    def free(self):
        if self.ptr is not None:
            self.gpu.free(self.ptr)
            self.ptr = None
