"""Python side of the HIP runtime (csrc/capi.hip, C ABI in include/h3hip.h).

Mirrors the reference's h3metal/gpu.py (:94-305): `Gpu` opens the device and
launches kernels, a `Tensor` is a typed view (buffer, byte offset, shape,
dtype) of a device buffer, `pack` builds parameter blocks. Kernels run on one
HIP stream in submission order; `Gpu.wait()` blocks and returns GPU seconds.

Deviation from the reference (documented, unavoidable on a discrete GPU): the
buffers are device memory, so `Tensor.numpy()` returns a host COPY (taken after
the stream drains) instead of a live view, and writing goes through
`Tensor.write()` / `Gpu.upload()` instead of assigning into `numpy()`.
"""

from __future__ import annotations

import ctypes
import math
import os
import struct
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libh3hip.so"


def _find_library() -> str:
    for c in (os.environ.get("H3HIP_LIB", ""), os.path.join(_HERE, LIB_NAME)):
        if c and os.path.exists(c):
            return os.path.abspath(c)
    raise FileNotFoundError(f"{LIB_NAME} not found next to {__file__}; build it with `python -m h3metal_amd.build`")


class _Arg(ctypes.Structure):
    _fields_ = [("buf", ctypes.c_void_p), ("offset", ctypes.c_uint64)]


# Every exported symbol of include/h3hip.h with its ctypes signature.
SIGNATURES = {
    "h3_last_error": (ctypes.c_char_p, []),
    "h3_open": (ctypes.c_void_p, [ctypes.c_char_p]),
    "h3_close": (None, [ctypes.c_void_p]),
    "h3_device_name": (ctypes.c_char_p, [ctypes.c_void_p]),
    "h3_recommended_working_set": (ctypes.c_uint64, [ctypes.c_void_p]),
    "h3_max_buffer_length": (ctypes.c_uint64, [ctypes.c_void_p]),
    "h3_buffer": (ctypes.c_void_p, [ctypes.c_void_p, ctypes.c_uint64]),
    "h3_buffer_contents": (ctypes.c_void_p, [ctypes.c_void_p]),
    "h3_buffer_length": (ctypes.c_uint64, [ctypes.c_void_p]),
    "h3_buffer_release": (None, [ctypes.c_void_p]),
    "h3_buffer_write": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                       ctypes.c_uint64]),
    "h3_buffer_read": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                      ctypes.c_uint64]),
    "h3_buffer_device": (ctypes.c_void_p, [ctypes.c_void_p]),
    "h3_pipeline": (ctypes.c_void_p, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p]),
    "h3_pipeline_max_threads": (ctypes.c_int, [ctypes.c_void_p]),
    "h3_dispatch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32),
                                   ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_Arg), ctypes.c_int,
                                   ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_uint32]),
    "h3_dispatch_static": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32),
                                          ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_Arg), ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_uint32]),
    "h3_commit": (None, [ctypes.c_void_p]),
    "h3_wait": (ctypes.c_double, [ctypes.c_void_p]),
    "h3_set_profile": (None, [ctypes.c_void_p, ctypes.c_int]),
    "h3_profile_take": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double), ctypes.c_int]),
    "h3_reserve_workspace": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint64]),
    "h3_workspace_bytes": (ctypes.c_uint64, [ctypes.c_void_p]),
}


def _load():
    lib = ctypes.CDLL(_find_library())
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


class GpuError(RuntimeError):
    pass


def _err() -> str:
    return lib().h3_last_error().decode()


_NP = {
    "f32": np.float32, "f16": np.float16, "bf16": np.uint16, "i8": np.int8, "u8": np.uint8,
    "i32": np.int32, "u32": np.uint32, "i16": np.int16, "u16": np.uint16,
}
_SIZE = {"f32": 4, "f16": 2, "bf16": 2, "i8": 1, "u8": 1, "i32": 4, "u32": 4, "i16": 2, "u16": 2}
_FROM_NP = {np.dtype(np.float32): "f32", np.dtype(np.float16): "f16", np.dtype(np.int8): "i8",
            np.dtype(np.uint8): "u8", np.dtype(np.int32): "i32", np.dtype(np.uint32): "u32",
            np.dtype(np.uint16): "bf16", np.dtype(np.int16): "i16"}


@dataclass
class Buffer:
    handle: int
    nbytes: int
    gpu: "Gpu" = None

    def __del__(self):
        if self.handle and _lib is not None:
            _lib.h3_buffer_release(self.handle)
            self.handle = 0


@dataclass
class Tensor:
    """Element type, shape and starting byte of some device memory inside a `Buffer`."""
    buf: Buffer
    offset: int
    shape: tuple
    dtype: str
    strides: tuple = field(default=None)  # in elements; None = contiguous

    @property
    def nbytes(self) -> int:
        return int(math.prod(self.shape) * _SIZE[self.dtype])

    def arg(self):
        return (self.buf.handle, self.offset)

    def numpy(self) -> np.ndarray:
        """A host copy of the data, taken after all queued GPU work has finished."""
        out = np.empty(self.shape, _NP[self.dtype])
        if out.nbytes:
            rc = lib().h3_buffer_read(self.buf.gpu.ctx, self.buf.handle, self.offset, out.ctypes.data, out.nbytes)
            if rc:
                raise GpuError(_err())
        return out

    def write(self, arr: np.ndarray, offset_elems: int = 0):
        """Copies `arr` (raw bytes of the tensor's element type) into the tensor, starting at an element offset."""
        a = np.ascontiguousarray(arr)
        if a.dtype != np.dtype(_NP[self.dtype]):
            a = a.astype(_NP[self.dtype])
        off = self.offset + int(offset_elems * _SIZE[self.dtype])
        if off + a.nbytes > self.offset + self.nbytes:
            raise GpuError(f"write of {a.nbytes} bytes at element {offset_elems} exceeds the tensor {self.shape}")
        if a.nbytes:
            rc = lib().h3_buffer_write(self.buf.gpu.ctx, self.buf.handle, off, a.ctypes.data, a.nbytes)
            if rc:
                raise GpuError(_err())

    def view(self, shape, dtype=None, offset_elems=0):
        dtype = dtype or self.dtype
        return Tensor(self.buf, self.offset + int(offset_elems * _SIZE[self.dtype]), tuple(shape), dtype)

    def row(self, start: int, count: int):
        """`count` leading-axis slices starting at slice `start`, for a tensor stored without gaps."""
        per = int(math.prod(self.shape[1:]))
        return Tensor(self.buf, self.offset + int(start * per * _SIZE[self.dtype]), (count,) + tuple(self.shape[1:]),
                      self.dtype)


class Kernel:
    """A kernel specialisation selected from the library's launch table."""

    def __init__(self, gpu: "Gpu", file: str, fn: str, macros: dict | None = None):
        ms = ";".join(f"{k}={v}" for k, v in sorted((macros or {}).items()))
        self.handle = lib().h3_pipeline(gpu.ctx, file.encode(), fn.encode(), ms.encode())
        if not self.handle:
            raise GpuError(_err())
        self.max_threads = lib().h3_pipeline_max_threads(self.handle)
        self.name = f"{file}:{fn}({ms})"


class Gpu:
    def __init__(self, kernel_dir: str | None = None):
        self.ctx = lib().h3_open((kernel_dir or "").encode())
        if not self.ctx:
            raise GpuError(_err())
        self.device = lib().h3_device_name(self.ctx).decode()
        self.working_set = lib().h3_recommended_working_set(self.ctx)
        self.max_buffer = lib().h3_max_buffer_length(self.ctx)
        self._kernels = {}
        self.names = []  # while profiling: one name per launch, matched with its duration by profile_take()

    def kernel(self, file: str, fn: str, **macros) -> Kernel:
        key = (file, fn, tuple(sorted(macros.items())))
        k = self._kernels.get(key)
        if k is None:
            k = Kernel(self, file, fn, macros)
            self._kernels[key] = k
        return k

    def buffer(self, nbytes: int) -> Buffer:
        h = lib().h3_buffer(self.ctx, max(1, int(nbytes)))
        if not h:
            raise GpuError(_err())
        return Buffer(h, int(nbytes), self)

    def empty(self, shape, dtype="f32") -> Tensor:
        """A zero-filled tensor (the reference's buffers are zero-filled too)."""
        shape = tuple(int(s) for s in shape)
        nbytes = int(math.ceil(math.prod(shape) * _SIZE[dtype]))
        return Tensor(self.buffer(nbytes), 0, shape, dtype)

    zeros = empty

    def upload(self, arr: np.ndarray, dtype: str | None = None) -> Tensor:
        if dtype is None:
            dtype = _FROM_NP[np.dtype(arr.dtype)]
        t = self.empty(arr.shape, dtype)
        t.write(np.ascontiguousarray(arr).view(_NP[dtype]).reshape(t.shape))
        return t

    def launch(self, k: Kernel, grid, threads, args, params: bytes = b"", params_index: int | None = None,
               tg_mem: int = 0, no_alloc: bool = False):
        """Launches kernel `k` with buffers `args` (Tensor, (Buffer, offset) or None) and a parameter block.
        grid / threads may be None: each gfx950 kernel chooses its own geometry from its parameters."""
        g = (ctypes.c_uint32 * 3)(*(list(grid or ()) + [0, 0, 0])[:3])
        t = (ctypes.c_uint32 * 3)(*(list(threads or ()) + [0, 0, 0])[:3])
        n = len(args)
        arr = (_Arg * max(1, n))()
        for i, a in enumerate(args):
            if a is None:
                arr[i].buf, arr[i].offset = None, 0
            elif isinstance(a, Tensor):
                arr[i].buf, arr[i].offset = a.buf.handle, a.offset
            else:  # (Buffer, offset)
                arr[i].buf, arr[i].offset = a[0].handle, a[1]
        pi = n if params_index is None else params_index
        pbuf = ctypes.create_string_buffer(params, len(params)) if params else None
        entry = lib().h3_dispatch_static if no_alloc else lib().h3_dispatch
        rc = entry(self.ctx, k.handle, g, t, arr, n, pbuf, len(params), pi, tg_mem)
        if rc:
            raise GpuError(_err())
        if self._profile:
            self.names.append(k.name)

    _profile = False

    def commit(self):
        lib().h3_commit(self.ctx)

    def wait(self) -> float:
        dt = lib().h3_wait(self.ctx)
        if dt < 0:
            raise GpuError(_err())
        return dt

    def profile(self, on: bool):
        lib().h3_set_profile(self.ctx, 1 if on else 0)
        self._profile = on
        self.names = []

    def profile_take(self):
        out = (ctypes.c_double * 100000)()
        n = lib().h3_profile_take(self.ctx, out, 100000)
        names, self.names = self.names[:n], self.names[n:]
        return list(zip(names, out[:n]))

    def reserve_workspace(self, nbytes: int):
        """Grows the dispatch scratch memory to at least `nbytes` (drains the stream first when it grows), so
        that a later launch needing that much scratch neither allocates nor waits."""
        if lib().h3_reserve_workspace(self.ctx, int(nbytes)):
            raise GpuError(_err())

    @property
    def workspace_bytes(self) -> int:
        return int(lib().h3_workspace_bytes(self.ctx))

    def close(self):
        if self.ctx:
            lib().h3_close(self.ctx)
            self.ctx = None


def pack(fmt: str, *vals) -> bytes:
    return struct.pack("<" + fmt, *vals)
