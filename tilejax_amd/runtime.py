"""The host side of the C-ABI (include/ak.h): compile generated HIP with hiprtc, load it, launch it.

This is the device boundary the reference reaches through `jax.jit(entry)` and `pl.pallas_call`
(src/autokernel/api.py:69-72, codegen.py:468-501). PyTorch allocates every buffer; the library borrows
raw pointers for a launch, on torch's current stream.

Code objects are cached on disk by a hash of (source, options): a build-speed measure, not a tuning cache
(tuning results live in memory only, as in the reference). `TILEJAX_CACHE` moves the cache.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import threading
from typing import Any, Dict, List, Optional, Sequence, Tuple

from . import gfx950
from .errors import KernelError

__all__ = ["Library", "compile_source", "library", "load", "Module", "spin"]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libak.so")
CACHE_DIR = os.environ.get("TILEJAX_CACHE", os.path.join(_HERE, "_cache"))
# Flags of every generated kernel: gfx950 only; packed-FP32 instructions off (a workaround this image's
# GPUs need); -O3.
OPTIONS = ("--offload-arch=" + gfx950.ARCH, "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")


class Library:
    """libak.so, loaded with ctypes; every call raises KernelError with the library's message on failure."""

    def __init__(self, path: str = LIB_PATH) -> None:
        if not os.path.exists(path):
            raise KernelError(f"the HIP runtime library {path} is not built: run __graft_entry__.build() first")
        self.path = path
        self.lib = ctypes.CDLL(path)
        L = self.lib
        vp, sz, i32, u32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint32
        L.ak_last_error.restype = ctypes.c_char_p
        L.ak_version.restype = i32
        L.ak_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(vp), ctypes.POINTER(sz)]
        L.ak_free.argtypes = [vp]
        L.ak_free.restype = None
        L.ak_device_count.restype = i32
        L.ak_module_load.argtypes = [vp, sz, ctypes.POINTER(vp)]
        L.ak_module_free.argtypes = [vp]
        L.ak_get_kernel.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(vp)]
        L.ak_kernel_info.argtypes = [vp] + [ctypes.POINTER(i32)] * 4
        L.ak_launch.argtypes = [vp, u32, u32, u32, u32, u32, u32, u32, vp, sz, vp]
        L.ak_launch_scratch.argtypes = [vp, u32, u32, u32, u32, u32, u32, u32, vp, sz, ctypes.POINTER(sz),
                                         ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64), sz, vp]
        L.ak_event_create.argtypes = [ctypes.POINTER(vp)]
        L.ak_event_record.argtypes = [vp, vp]
        L.ak_event_elapsed_ms.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_float)]
        L.ak_event_destroy.argtypes = [vp]
        L.ak_stream_synchronize.argtypes = [vp]
        for name in ("ak_compile", "ak_module_load", "ak_module_free", "ak_get_kernel", "ak_kernel_info", "ak_launch",
                     "ak_launch_scratch",
                     "ak_event_create", "ak_event_record", "ak_event_elapsed_ms", "ak_event_destroy",
                     "ak_stream_synchronize"):
            getattr(L, name).restype = i32

    def check(self, status: int, what: str) -> None:
        if status != 0:
            message = self.lib.ak_last_error().decode(errors="replace")
            raise KernelError(f"{what}: {message}")

    def compile(self, source: str, name: str, options: Sequence[str] = OPTIONS) -> bytes:
        code, size = ctypes.c_void_p(), ctypes.c_size_t()
        opts = b"".join(o.encode() + b"\0" for o in options) + b"\0"
        self.check(self.lib.ak_compile(source.encode(), name.encode(), opts, ctypes.byref(code), ctypes.byref(size)),
                   f"compiling {name} for {gfx950.ARCH}")
        try:
            return ctypes.string_at(code, size.value)
        finally:
            self.lib.ak_free(code)

    def device_count(self) -> int:
        return int(self.lib.ak_device_count())


_LIBRARY: Optional[Library] = None
_LOCK = threading.Lock()


def library() -> Library:
    global _LIBRARY
    with _LOCK:
        if _LIBRARY is None:
            _LIBRARY = Library()
        return _LIBRARY


def compile_source(source: str, name: str, options: Sequence[str] = OPTIONS) -> bytes:
    """The gfx950 code object of `source`, from the cache or compiled now."""
    key = hashlib.sha256(("\0".join(options) + "\0" + source).encode()).hexdigest()[:32]
    path = os.path.join(CACHE_DIR, f"{key}.hsaco")
    if os.path.exists(path):
        with open(path, "rb") as f:
            return f.read()
    code = library().compile(source, name, options)
    try:
        os.makedirs(CACHE_DIR, exist_ok=True)
        tmp = f"{path}.{os.getpid()}.tmp"
        with open(tmp, "wb") as f:
            f.write(code)
        os.replace(tmp, path)
    except OSError:
        pass  # a read-only tree: the code object just isn't cached
    return code


class Kernel:
    """One __global__ function of a loaded module."""

    def __init__(self, module: "Module", symbol: str) -> None:
        lib = library()
        handle = ctypes.c_void_p()
        lib.check(lib.lib.ak_get_kernel(module.handle, symbol.encode(), ctypes.byref(handle)), f"kernel {symbol}")
        self.module, self.symbol, self.handle = module, symbol, handle

    def info(self) -> Dict[str, int]:
        vals = [ctypes.c_int(-1) for _ in range(4)]
        library().check(library().lib.ak_kernel_info(self.handle, *[ctypes.byref(v) for v in vals]), "kernel info")
        return dict(zip(("vgprs", "lds_bytes", "private_bytes", "max_threads"), (v.value for v in vals)))

    def launch(self, grid: Tuple[int, int, int], block: Tuple[int, int, int], lds: int, args: bytes, stream: int) -> None:
        lib = library()
        buf = ctypes.create_string_buffer(args, len(args))
        lib.check(lib.lib.ak_launch(self.handle, grid[0], grid[1], grid[2], block[0], block[1], block[2], lds,
                                    ctypes.cast(buf, ctypes.c_void_p), len(args), ctypes.c_void_p(stream)),
                  f"launching {self.symbol}")


    def launch_scratch(self, grid: Tuple[int, int, int], block: Tuple[int, int, int], lds: int, args: bytes,
                       stream: int, placed: Sequence[Tuple[int, int, int]]) -> None:
        """Launch with the workspace pointer fields of `args` placed in the library's scratch array:
        `placed` lists (byte offset of the field in args, offset in the scratch array, bytes). Allocates
        nothing on the device (include/ak.h, ak_launch_scratch)."""
        lib = library()
        buf = ctypes.create_string_buffer(args, len(args))
        n = len(placed)
        fields = (ctypes.c_size_t * max(n, 1))(*(p[0] for p in placed))
        offsets = (ctypes.c_uint64 * max(n, 1))(*(p[1] for p in placed))
        sizes = (ctypes.c_uint64 * max(n, 1))(*(p[2] for p in placed))
        lib.check(lib.lib.ak_launch_scratch(self.handle, grid[0], grid[1], grid[2], block[0], block[1], block[2],
                                            lds, ctypes.cast(buf, ctypes.c_void_p), len(args), fields, offsets,
                                            sizes, n, ctypes.c_void_p(stream)),
                  f"launching {self.symbol} on the library's scratch")


# The library's scratch array per device (include/ak.h AK_SCRATCH_BYTES), and the alignment of each
# workspace buffer placed in it.
SCRATCH_BYTES = 64 << 20
SCRATCH_ALIGN = 256


class Module:
    """A loaded code object."""

    def __init__(self, code: bytes) -> None:
        lib = library()
        handle = ctypes.c_void_p()
        self._code = ctypes.create_string_buffer(code, len(code))
        lib.check(lib.lib.ak_module_load(ctypes.cast(self._code, ctypes.c_void_p), len(code), ctypes.byref(handle)),
                  "loading a gfx950 code object")
        self.handle = handle
        self.kernels: Dict[str, Kernel] = {}

    def kernel(self, symbol: str) -> Kernel:
        if symbol not in self.kernels:
            self.kernels[symbol] = Kernel(self, symbol)
        return self.kernels[symbol]


def load(source: str, name: str) -> Module:
    """Compile (or find in the cache) and load `source` on the current device."""
    return Module(compile_source(source, name))


class Event:
    """A HIP event on a stream, for device time."""

    def __init__(self) -> None:
        handle = ctypes.c_void_p()
        library().check(library().lib.ak_event_create(ctypes.byref(handle)), "hipEventCreate")
        self.handle = handle

    def record(self, stream: int) -> None:
        library().check(library().lib.ak_event_record(self.handle, ctypes.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float()
        library().check(library().lib.ak_event_elapsed_ms(self.handle, later.handle, ctypes.byref(ms)), "elapsed")
        return float(ms.value)

    def __del__(self) -> None:
        try:
            library().lib.ak_event_destroy(self.handle)
        except Exception:
            pass


# A one-wave kernel that waits `ticks` of the 100 MHz constant clock, then exits: queued ahead of timed
# calls, it holds the GPU while the host launches them all, so the host's launch time never shows up as
# gaps between them.
_SPIN_SOURCE = r"""
extern "C" __global__ void __launch_bounds__(64) ak_spin(const unsigned long long ticks) {
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(32);
}
"""
_SPIN: Dict[int, "Kernel"] = {}
SPIN_MAX_S = 0.05


def spin(seconds: float, stream: int) -> None:
    """Queue a kernel on `stream` that keeps the GPU waiting for `seconds` (at most SPIN_MAX_S)."""
    import struct

    import torch

    device = torch.cuda.current_device()
    if device not in _SPIN:
        _SPIN[device] = load(_SPIN_SOURCE, "ak_spin.hip").kernel("ak_spin")
    ticks = int(min(max(seconds, 0.0), SPIN_MAX_S) * 100e6)
    _SPIN[device].launch((1, 1, 1), (64, 1, 1), 0, struct.pack("<Q", ticks), stream)


def current_stream() -> int:
    """torch's current HIP stream, as the raw handle kernels launch on."""
    import torch

    return int(torch.cuda.current_stream().cuda_stream)


def require_gpu() -> None:
    """Kernels run on a GPU only: there is no CPU fallback."""
    import torch

    if not torch.cuda.is_available():
        raise KernelError("tilejax_amd kernels run on an MI355X (gfx950): no GPU is visible")
