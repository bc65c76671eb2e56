"""Python side of the HIP runtime: a ctypes binding of the C ABI in include/h3hip.h (csrc/capi.hip).

The public names and their meaning are those of the reference's runtime module (h3metal/gpu.py:94-305), so
that the launchers in ops.py and the reference's callers run unchanged: `Gpu` opens the device, selects kernels
and launches them in submission order on one stream; `Tensor` is a typed view (buffer, byte offset, shape,
dtype) of a device `Buffer`; `pack` builds parameter blocks; `Gpu.wait()` blocks and returns GPU seconds.

Deviation (a discrete GPU has no shared memory): `Tensor.numpy()` returns a host copy taken after the stream
drains, and data goes in through `Tensor.write()` / `Gpu.upload()`; `Tensor.copy_to()` copies on the device.
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


class GpuError(RuntimeError):
    pass


def _find_library() -> str:
    """H3HIP_LIB if set, else the library built next to this file (python -m h3metal_amd.build)."""
    for path in (os.environ.get("H3HIP_LIB", ""), os.path.join(_HERE, LIB_NAME)):
        if path and os.path.exists(path):
            return os.path.abspath(path)
    raise FileNotFoundError(f"{LIB_NAME} not found next to {__file__}; build it with `python -m h3metal_amd.build`")


class _Arg(ctypes.Structure):  # h3_arg
    _fields_ = [("buf", ctypes.c_void_p), ("offset", ctypes.c_uint64)]


_P, _U64, _U32, _I = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
_DISPATCH = (_I, [_P, _P, ctypes.POINTER(_U32), ctypes.POINTER(_U32), ctypes.POINTER(_Arg), _I, _P, _U32, _I, _U32])

# Every exported symbol of include/h3hip.h: (result type, argument types).
SIGNATURES = {
    "h3_last_error": (ctypes.c_char_p, []),
    "h3_open": (_P, [ctypes.c_char_p]),
    "h3_close": (None, [_P]),
    "h3_device_name": (ctypes.c_char_p, [_P]),
    "h3_recommended_working_set": (_U64, [_P]),
    "h3_max_buffer_length": (_U64, [_P]),
    "h3_buffer": (_P, [_P, _U64]),
    "h3_buffer_contents": (_P, [_P]),
    "h3_buffer_length": (_U64, [_P]),
    "h3_buffer_release": (None, [_P]),
    "h3_buffer_write": (_I, [_P, _P, _U64, _P, _U64]),
    "h3_buffer_read": (_I, [_P, _P, _U64, _P, _U64]),
    "h3_buffer_copy": (_I, [_P, _P, _U64, _P, _U64, _U64]),
    "h3_buffer_device": (_P, [_P]),
    "h3_pipeline": (_P, [_P, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p]),
    "h3_pipeline_max_threads": (_I, [_P]),
    "h3_dispatch": _DISPATCH,
    "h3_dispatch_static": _DISPATCH,
    "h3_commit": (None, [_P]),
    "h3_wait": (ctypes.c_double, [_P]),
    "h3_set_profile": (None, [_P, _I]),
    "h3_profile_take": (_I, [_P, ctypes.POINTER(ctypes.c_double), _I]),
    "h3_reserve_workspace": (_I, [_P, _U64]),
    "h3_workspace_bytes": (_U64, [_P]),
}

_native = None


def lib():
    """The loaded library, every symbol of SIGNATURES typed (loaded on first use)."""
    global _native
    if _native is None:
        handle = ctypes.CDLL(_find_library())
        for name, (res, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, argtypes
        _native = handle
    return _native


def _call(name: str, *args, fails=lambda r: r != 0):
    """Calls C function `name`; raises GpuError with the library's thread-local message when `fails(result)`."""
    r = getattr(lib(), name)(*args)
    if fails(r):
        raise GpuError(lib().h3_last_error().decode())
    return r


_NULL = lambda r: not r  # noqa: E731 -- handle-returning calls fail with NULL

# element type name -> (numpy dtype of its raw bytes, bytes per element); "bf16" travels as uint16 bit patterns
_DT = {"f32": (np.float32, 4), "f16": (np.float16, 2), "bf16": (np.uint16, 2), "i8": (np.int8, 1),
       "u8": (np.uint8, 1), "i32": (np.int32, 4), "u32": (np.uint32, 4), "i16": (np.int16, 2),
       "u16": (np.uint16, 2)}
_BY_NUMPY = {np.dtype(np.float32): "f32", np.dtype(np.float16): "f16", np.dtype(np.int8): "i8",
             np.dtype(np.uint8): "u8", np.dtype(np.int32): "i32", np.dtype(np.uint32): "u32",
             np.dtype(np.uint16): "bf16", np.dtype(np.int16): "i16"}


@dataclass
class Buffer:
    """One device allocation (h3_buffer); released when the object goes away."""
    handle: int
    nbytes: int
    gpu: "Gpu" = None

    def __del__(self):
        if self.handle and _native is not None:
            _native.h3_buffer_release(self.handle)
        self.handle = 0


@dataclass
class Tensor:
    """`shape` elements of type `dtype` stored from byte `offset` of `buf` (row-major unless `strides` says
    otherwise, in elements)."""
    buf: Buffer
    offset: int
    shape: tuple
    dtype: str
    strides: tuple = field(default=None)

    @property
    def itemsize(self) -> int:
        return _DT[self.dtype][1]

    @property
    def nbytes(self) -> int:
        return int(math.prod(self.shape) * self.itemsize)

    def arg(self):
        """The (buffer handle, byte offset) pair a dispatch binds."""
        return (self.buf.handle, self.offset)

    def _ctx(self):
        return self.buf.gpu.ctx

    def numpy(self) -> np.ndarray:
        """A host copy of the data, taken after all queued GPU work has finished."""
        host = np.empty(self.shape, _DT[self.dtype][0])
        if host.nbytes:
            _call("h3_buffer_read", self._ctx(), self.buf.handle, self.offset, host.ctypes.data, host.nbytes)
        return host

    def write(self, arr: np.ndarray, offset_elems: int = 0):
        """Copies `arr` (converted to this tensor's raw element type) in, starting `offset_elems` elements in."""
        data = np.ascontiguousarray(arr, dtype=_DT[self.dtype][0])
        start = int(offset_elems * self.itemsize)
        if start + data.nbytes > self.nbytes:
            raise GpuError(f"write of {data.nbytes} bytes at element {offset_elems} exceeds the tensor {self.shape}")
        if data.nbytes:
            _call("h3_buffer_write", self._ctx(), self.buf.handle, self.offset + start, data.ctypes.data, data.nbytes)

    def copy_to(self, dst: "Tensor", nbytes: int | None = None):
        """Queues a device-to-device copy of this tensor's bytes (or the first `nbytes`) into `dst`, in order with
        the launches of the context."""
        n = self.nbytes if nbytes is None else int(nbytes)
        _call("h3_buffer_copy", self._ctx(), dst.buf.handle, dst.offset, self.buf.handle, self.offset, n)
        if n and self.buf.gpu._profile:  # timed like a launch
            self.buf.gpu.names.append("h3_buffer_copy")

    def view(self, shape, dtype=None, offset_elems=0):
        """Another shape / type over the same bytes, starting `offset_elems` elements (of this type) in."""
        return Tensor(self.buf, self.offset + int(offset_elems * self.itemsize), tuple(shape), dtype or self.dtype)

    def row(self, start: int, count: int):
        """`count` leading-axis slices from slice `start`, for a tensor stored without gaps."""
        inner = tuple(self.shape[1:])
        return self.view((count,) + inner, offset_elems=start * int(math.prod(inner)))


class Kernel:
    """A kernel specialisation of the library's launch table (h3_pipeline)."""

    def __init__(self, gpu: "Gpu", file: str, fn: str, macros: dict | None = None):
        spec = ";".join(f"{k}={v}" for k, v in sorted((macros or {}).items()))
        self.handle = _call("h3_pipeline", gpu.ctx, file.encode(), fn.encode(), spec.encode(), fails=_NULL)
        self.max_threads = lib().h3_pipeline_max_threads(self.handle)
        self.name = f"{file}:{fn}({spec})"


def _bind(args) -> tuple:
    """The h3_arg array of a launch: a Tensor binds (its buffer, its offset), a (Buffer, offset) pair binds that,
    None binds nothing (a NULL buffer)."""
    arr = (_Arg * max(1, len(args)))()
    for slot, a in zip(arr, args):
        if isinstance(a, Tensor):
            slot.buf, slot.offset = a.buf.handle, a.offset
        elif a is not None:
            slot.buf, slot.offset = a[0].handle, a[1]
    return arr, len(args)


def _dims(v):
    return (_U32 * 3)(*(tuple(v or ()) + (0, 0, 0))[:3])


class Gpu:
    """One device context: a HIP stream, its kernels and buffers."""

    def __init__(self, kernel_dir: str | None = None):
        self.ctx = _call("h3_open", (kernel_dir or "").encode(), fails=_NULL)
        self.device = lib().h3_device_name(self.ctx).decode()
        self.working_set = lib().h3_recommended_working_set(self.ctx)
        self.max_buffer = lib().h3_max_buffer_length(self.ctx)
        self._kernels = {}
        self._profile = False
        self.names = []  # in profile mode: the kernel name of each timed launch, in order, until profile_take()

    def kernel(self, file: str, fn: str, **macros) -> Kernel:
        key = (file, fn, tuple(sorted(macros.items())))
        if key not in self._kernels:
            self._kernels[key] = Kernel(self, file, fn, macros)
        return self._kernels[key]

    def buffer(self, nbytes: int) -> Buffer:
        return Buffer(_call("h3_buffer", self.ctx, max(1, int(nbytes)), fails=_NULL), int(nbytes), self)

    def empty(self, shape, dtype="f32") -> Tensor:
        """A zero-filled tensor (the reference's buffers are zero-filled too)."""
        shape = tuple(int(s) for s in shape)
        return Tensor(self.buffer(int(math.ceil(math.prod(shape) * _DT[dtype][1]))), 0, shape, dtype)

    zeros = empty

    def upload(self, arr: np.ndarray, dtype: str | None = None) -> Tensor:
        dtype = dtype or _BY_NUMPY[np.dtype(arr.dtype)]
        t = self.empty(arr.shape, dtype)
        t.write(np.ascontiguousarray(arr).view(_DT[dtype][0]).reshape(t.shape))
        return t

    def launch(self, k: Kernel, grid, threads, args, params: bytes = b"", params_index: int | None = None,
               tg_mem: int = 0, no_alloc: bool = False):
        """Queues kernel `k` with buffers `args` (Tensor, (Buffer, offset) or None) and a parameter block placed at
        `params_index` (default: after the buffers). grid / threads may be None: each gfx950 kernel chooses its own
        geometry from its parameters. no_alloc: the allocation-free entry point (h3_dispatch_static), which uses
        the library's fixed scratch array and is not timed per launch."""
        arr, n = _bind(args)
        block = ctypes.create_string_buffer(params, len(params)) if params else None
        entry = "h3_dispatch_static" if no_alloc else "h3_dispatch"
        _call(entry, self.ctx, k.handle, _dims(grid), _dims(threads), arr, n, block, len(params),
              n if params_index is None else params_index, tg_mem)
        if self._profile and not no_alloc:
            self.names.append(k.name)

    def commit(self):
        lib().h3_commit(self.ctx)

    def wait(self) -> float:
        """Blocks until the queued work is done; GPU seconds since the first launch after the previous wait."""
        return _call("h3_wait", self.ctx, fails=lambda r: r < 0)

    def profile(self, on: bool):
        """Per-launch timing on or off (drains the stream; forgets what was not taken)."""
        lib().h3_set_profile(self.ctx, 1 if on else 0)
        self._profile = on
        self.names = []

    def profile_take(self):
        """(kernel name, seconds) of the timed launches since the last take, in submission order."""
        out = (ctypes.c_double * max(1, len(self.names)))()
        n = lib().h3_profile_take(self.ctx, out, len(out))
        taken, self.names = self.names[:n], self.names[n:]
        return list(zip(taken, out[:n]))

    def reserve_workspace(self, nbytes: int):
        """Grows the dispatch scratch memory to at least `nbytes` (drains the stream first when it grows), so
        that a later launch needing that much scratch neither allocates nor waits."""
        _call("h3_reserve_workspace", self.ctx, int(nbytes))

    @property
    def workspace_bytes(self) -> int:
        return int(lib().h3_workspace_bytes(self.ctx))

    def close(self):
        if self.ctx:
            lib().h3_close(self.ctx)
            self.ctx = None


def pack(fmt: str, *vals) -> bytes:
    """A little-endian parameter block (struct format `fmt`)."""
    return struct.pack("<" + fmt, *vals)
