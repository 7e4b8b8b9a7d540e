"""mcke_amd -- the MI355X (gfx950) MCKE kernel layer, host side.

A thin ctypes mirror of the reference's C++ kernel and runtime interface over the
C-ABI in ``include/mcke_amd.h`` (library: ``lib/libmcke_amd.so``):

* ``launch_*_f32`` keep the names, argument order and meaning of
  ``mcke::kernels::launch_*_f32`` (reference include/mcke/kernels/kernels.hpp) and
  return a :class:`Status` (reference include/mcke/core/status.hpp) instead of
  raising, so callers check ``.ok()`` exactly as the reference's benches do;
* :class:`Stream`, :class:`Event` mirror ``rt::Stream`` / ``rt::Event``
  (reference include/mcke/runtime/stream.hpp:82-306);
* :class:`DeviceBuffer` is a raw device allocation (``RawDeviceAllocator``,
  reference src/memory/allocator.cpp:44-73) with host upload/download.

There is no CPU fallback: every launch runs the HIP kernels in the library, and
loading fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmcke_amd.so")

# ---------------------------------------------------------------------------
# Vocabulary (numeric values are the reference's and are ABI)
# ---------------------------------------------------------------------------


class StatusCode(enum.IntEnum):          # status.hpp:42-50
    kOk = 0
    kOutOfMemory = 1
    kInvalidArgument = 2
    kFailedPrecondition = 3
    kUnimplemented = 4
    kInternal = 5
    kDeviceError = 6                     # the reference's kCudaError slot


class Activation(enum.IntEnum):          # kernels.hpp:65
    kNone = 0
    kRelu = 1
    kGeluErf = 2
    kGeluTanh = 3


class ReduceKind(enum.IntEnum):          # kernels.hpp:153
    kSum = 0
    kMax = 1
    kMean = 2


class ReduceVariant(enum.IntEnum):       # kernels.hpp:180
    kSmemTree = 0
    kWarpShuffle = 1
    kTwoPass = 2


class SoftmaxVariant(enum.IntEnum):      # kernels.hpp:218
    kThreePass = 0
    kOnlineOnePass = 1


class GemmVariant(enum.IntEnum):         # gemm_tile.hpp:209-214, append-only
    kNaive = 0
    kTiledSmem = 1
    kTiledRegBlock = 2
    kWarpTile = 3
    kCublasRef = 4
    kWarpTileNoDbuf = 5
    kWarpTileVec4 = 6
    kNaiveUncoalesced = 7
    kMfmaF32 = 8                         # appended: fp32 MFMA (gfx950)


class DType(enum.IntEnum):               # include/mcke/core/dtype.hpp:33-41 (first three)
    kF32 = 0
    kF16 = 1
    kBF16 = 2


class GemmTile(C.Structure):             # gemm_tile.hpp:47-69
    _fields_ = [("bm", C.c_int32), ("bn", C.c_int32), ("bk", C.c_int32),
                ("tm", C.c_int32), ("tn", C.c_int32)]

    def __init__(self, bm=128, bn=128, bk=8, tm=8, tn=8):
        super().__init__(bm, bn, bk, tm, tn)

    def __repr__(self):
        return f"GemmTile({self.bm},{self.bn},{self.bk},{self.tm},{self.tn})"

    def astuple(self):
        return (self.bm, self.bn, self.bk, self.tm, self.tn)


class KernelAttrs(C.Structure):          # kernels.hpp:293-299
    _fields_ = [("regs_per_thread", C.c_int32), ("agprs_per_thread", C.c_int32),
                ("static_smem_bytes", C.c_uint64), ("local_bytes", C.c_uint64),
                ("threads_per_block", C.c_int32), ("max_blocks_per_sm_api", C.c_int32)]


class DeviceInfo(C.Structure):           # device.hpp:29-110
    _fields_ = [("ordinal", C.c_int32), ("name", C.c_char * 256), ("arch", C.c_char * 64),
                ("cc_major", C.c_int32), ("cc_minor", C.c_int32),
                ("total_global_mem", C.c_uint64), ("sm_count", C.c_int32),
                ("warp_size", C.c_int32), ("max_threads_per_block", C.c_int32),
                ("max_threads_per_sm", C.c_int32), ("max_blocks_per_sm", C.c_int32),
                ("regs_per_block", C.c_int32), ("regs_per_sm", C.c_int32),
                ("shared_mem_per_block", C.c_uint64), ("shared_mem_per_sm", C.c_uint64),
                ("clock_khz", C.c_int32), ("memory_clock_khz", C.c_int32),
                ("memory_bus_width_bits", C.c_int32), ("l2_cache_bytes", C.c_uint64),
                ("peak_dram_gb_s", C.c_double)]


@dataclass(frozen=True)
class Status:
    """mcke::Status: a code plus a message (empty when OK)."""

    code: StatusCode = StatusCode.kOk
    message: str = ""

    def ok(self) -> bool:
        return self.code == StatusCode.kOk

    def __bool__(self) -> bool:          # truthiness == ok(), for `assert st`
        return self.ok()

    def __str__(self) -> str:
        return "Ok" if self.ok() else f"{self.code.name[1:]}: {self.message}"

    def throw_if_error(self) -> None:
        if not self.ok():
            raise MckeError(self)


class MckeError(RuntimeError):
    def __init__(self, status: Status):
        super().__init__(str(status))
        self.status = status


# ---------------------------------------------------------------------------
# Library loading
# ---------------------------------------------------------------------------
_lib = None
_VP = C.c_void_p
_I64 = C.c_int64


def library_path() -> str:
    return LIB_PATH


def lib() -> C.CDLL:
    """The loaded libmcke_amd.so.  Raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            f"g.build()'` (or `make -C {HERE}`).  There is no CPU fallback.")
    L = C.CDLL(LIB_PATH)
    sig = {
        "mcke_last_error": (C.c_char_p, []),
        "mcke_abi_version": (C.c_int, []),
        "mcke_launch_vector_add_f32": (C.c_int, [_VP, _VP, _VP, C.c_size_t, _VP]),
        "mcke_launch_bias_act_f32": (C.c_int, [_VP, _VP, _VP, _I64, _I64, C.c_int, C.c_int,
                                               _VP, C.c_int]),
        "mcke_launch_bias_add_f32": (C.c_int, [_VP, _VP, _VP, _I64, _I64, C.c_int, _VP]),
        "mcke_launch_activation_f32": (C.c_int, [_VP, _VP, _I64, C.c_int, C.c_int, _VP]),
        "mcke_max_vector_width_f32": (C.c_int, [_VP, _I64]),
        "mcke_row_reduce_workspace_bytes": (C.c_size_t, [_I64, _I64, C.c_int]),
        "mcke_launch_row_reduce_f32": (C.c_int, [_VP, _VP, _I64, _I64, C.c_int, C.c_int, _VP]),
        "mcke_launch_row_reduce_ws_f32": (C.c_int, [_VP, _VP, _I64, _I64, C.c_int, C.c_int,
                                                    _VP, C.c_size_t, _VP]),
        "mcke_launch_row_reduce_noalloc_f32": (C.c_int, [_VP, _VP, _I64, _I64, C.c_int, _VP]),
        "mcke_launch_row_softmax_f32": (C.c_int, [_VP, _VP, _I64, _I64, C.c_int, _VP]),
        "mcke_launch_gemm_f32": (C.c_int, [_VP, _VP, _VP, _I64, _I64, _I64, C.c_float,
                                           C.c_float, C.c_int, C.POINTER(GemmTile), _VP]),
        "mcke_launch_gemm_bias_act_f32": (C.c_int, [_VP, _VP, _VP, _VP, _I64, _I64, _I64,
                                                    C.c_float, C.c_int, C.POINTER(GemmTile),
                                                    _VP]),
        "mcke_gemm_kernel_attrs": (C.c_int, [C.c_int, C.POINTER(GemmTile),
                                             C.POINTER(KernelAttrs)]),
        "mcke_gemm_mfma_default_tile": (C.c_int, [_I64, _I64, _I64, C.POINTER(GemmTile)]),
        "mcke_launch_gemm_lp": (C.c_int, [_VP, _VP, _VP, C.c_int, C.c_int, _I64, _I64, _I64,
                                          C.c_float, C.c_float, C.POINTER(GemmTile), _VP]),
        "mcke_gemm_lp_kernel_attrs": (C.c_int, [C.c_int, C.c_int, C.POINTER(GemmTile),
                                                C.POINTER(KernelAttrs)]),
        "mcke_gemm_lp_default_tile": (C.c_int, [_I64, _I64, _I64, C.POINTER(GemmTile)]),
        "mcke_launch_gemm_lp_vendor": (C.c_int, [_VP, _VP, _VP, C.c_int, C.c_int, _I64, _I64,
                                                 _I64, C.c_float, C.c_float, _VP]),
        "mcke_rt_get_device_count": (C.c_int, [C.POINTER(C.c_int)]),
        "mcke_rt_set_device": (C.c_int, [C.c_int]),
        "mcke_rt_get_device": (C.c_int, [C.POINTER(C.c_int)]),
        "mcke_rt_query_device": (C.c_int, [C.c_int, C.POINTER(DeviceInfo)]),
        "mcke_rt_device_synchronize": (C.c_int, []),
        "mcke_rt_stream_create": (C.c_int, [C.POINTER(_VP)]),
        "mcke_rt_stream_destroy": (C.c_int, [_VP]),
        "mcke_rt_stream_synchronize": (C.c_int, [_VP]),
        "mcke_rt_stream_query": (C.c_int, [_VP, C.POINTER(C.c_int)]),
        "mcke_rt_stream_wait_event": (C.c_int, [_VP, _VP]),
        "mcke_rt_event_create": (C.c_int, [C.POINTER(_VP), C.c_int]),
        "mcke_rt_event_destroy": (C.c_int, [_VP]),
        "mcke_rt_event_record": (C.c_int, [_VP, _VP]),
        "mcke_rt_event_query": (C.c_int, [_VP, C.POINTER(C.c_int)]),
        "mcke_rt_event_synchronize": (C.c_int, [_VP]),
        "mcke_rt_event_elapsed_ms": (C.c_int, [_VP, _VP, C.POINTER(C.c_float)]),
        "mcke_rt_malloc": (C.c_int, [C.POINTER(_VP), C.c_size_t]),
        "mcke_rt_free": (C.c_int, [_VP]),
        "mcke_rt_host_alloc": (C.c_int, [C.POINTER(_VP), C.c_size_t]),
        "mcke_rt_host_free": (C.c_int, [_VP]),
        "mcke_rt_memcpy_async": (C.c_int, [_VP, _VP, C.c_size_t, C.c_int, _VP]),
        "mcke_rt_memset_async": (C.c_int, [_VP, C.c_int, C.c_size_t, _VP]),
        "mcke_mfma_peak_flops": (C.c_uint64, [_I64, _I64]),
        "mcke_launch_mfma_peak_f32": (C.c_int, [_VP, _VP, _I64, _I64, _VP]),
        "mcke_launch_stream_copy_f32": (C.c_int, [_VP, _VP, _I64, _VP]),
        "mcke_mfma_peak_lp_flops": (C.c_uint64, [_I64, _I64]),
        "mcke_launch_mfma_peak_lp": (C.c_int, [C.c_int, _VP, _VP, _I64, _I64, _VP]),
        "mcke_mfma_clock_lp_flops": (C.c_uint64, [_I64, _I64]),
        "mcke_launch_mfma_clock_lp": (C.c_int, [C.c_int, C.c_int, _VP, _VP, _VP, _I64, _I64, _VP]),
        "mcke_launch_stream_triad_f32": (C.c_int, [_VP, _VP, _VP, C.c_float, _I64, _VP]),
        "mcke_fill_random_f32": (None, [_VP, C.c_size_t, C.c_uint64, C.c_float, C.c_float]),
        "mcke_fill_normal_f32": (None, [_VP, C.c_size_t, C.c_uint64, C.c_float, C.c_float]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def exported_symbols() -> list[str]:
    """Every entry point this module binds (the C-ABI surface)."""
    lib()
    return sorted(n for n in dir(_lib) if n.startswith("mcke_"))


def _st(rc: int) -> Status:
    if rc == 0:
        return Status()
    msg = lib().mcke_last_error()
    return Status(StatusCode(rc), msg.decode() if msg else "")


def _ptr(p) -> int | None:
    """Device pointer from a DeviceBuffer, an int, or None."""
    if p is None:
        return None
    if isinstance(p, DeviceBuffer):
        return p.ptr
    if hasattr(p, "data_ptr"):           # a torch tensor on the GPU
        return int(p.data_ptr())
    return int(p)


def _sh(stream) -> int | None:
    if stream is None:
        return None
    if isinstance(stream, Stream):
        return stream.handle
    return int(stream)


def _check(rc: int) -> None:
    _st(rc).throw_if_error()


# ---------------------------------------------------------------------------
# Runtime: devices, streams, events, memory
# ---------------------------------------------------------------------------
def device_count() -> int:
    n = C.c_int(0)
    _check(lib().mcke_rt_get_device_count(C.byref(n)))
    return n.value


def query_device(ordinal: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    _check(lib().mcke_rt_query_device(ordinal, C.byref(info)))
    return info


def set_device(ordinal: int) -> None:
    _check(lib().mcke_rt_set_device(ordinal))


def device_synchronize() -> None:
    _check(lib().mcke_rt_device_synchronize())


def require_gpu() -> DeviceInfo:
    """Fails loudly unless a gfx950 GPU is visible (there is no CPU fallback)."""
    n = device_count()
    if n < 1:
        raise RuntimeError("no HIP device visible: the MCKE kernel layer needs an MI355X")
    info = query_device(0)
    if not info.arch.decode().startswith("gfx950"):
        raise RuntimeError(f"device 0 is {info.arch.decode()}, this build targets gfx950")
    set_device(0)
    return info


class Stream:
    """rt::Stream: an owned, non-blocking HIP stream (stream.hpp:132-148)."""

    def __init__(self):
        h = _VP()
        _check(lib().mcke_rt_stream_create(C.byref(h)))
        self.handle = h.value

    def synchronize(self) -> None:
        _check(lib().mcke_rt_stream_synchronize(self.handle))

    def query(self) -> bool:
        d = C.c_int(0)
        _check(lib().mcke_rt_stream_query(self.handle, C.byref(d)))
        return bool(d.value)

    def wait(self, event: "Event") -> None:
        _check(lib().mcke_rt_stream_wait_event(self.handle, event.handle))

    def close(self) -> None:
        if self.handle:
            lib().mcke_rt_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    """rt::Event (stream.hpp:196-306); timing events by default."""

    def __init__(self, timing: bool = True):
        h = _VP()
        _check(lib().mcke_rt_event_create(C.byref(h), 1 if timing else 0))
        self.handle = h.value

    def record(self, stream: Stream | None = None) -> None:
        _check(lib().mcke_rt_event_record(self.handle, _sh(stream)))

    def synchronize(self) -> None:
        _check(lib().mcke_rt_event_synchronize(self.handle))

    def query(self) -> bool:
        d = C.c_int(0)
        _check(lib().mcke_rt_event_query(self.handle, C.byref(d)))
        return bool(d.value)

    def elapsed_ms(self, stop: "Event") -> float:
        ms = C.c_float(0.0)
        _check(lib().mcke_rt_event_elapsed_ms(self.handle, stop.handle, C.byref(ms)))
        return ms.value

    def close(self) -> None:
        if self.handle:
            lib().mcke_rt_event_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """One hipMalloc'd region (RawDeviceAllocator semantics: 256-byte aligned)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _VP()
        _check(lib().mcke_rt_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, arr: np.ndarray, stream: Stream | None = None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr, stream)
        return buf

    @classmethod
    def zeros(cls, nfloats: int, stream: Stream | None = None) -> "DeviceBuffer":
        buf = cls(nfloats * 4)
        buf.memset(0, stream)
        return buf

    def upload(self, arr: np.ndarray, stream: Stream | None = None) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes, "upload larger than the buffer"
        _check(lib().mcke_rt_memcpy_async(self.ptr, arr.ctypes.data, arr.nbytes, 0, _sh(stream)))
        # pageable host memory: make the copy complete before `arr` can be freed
        _check(lib().mcke_rt_stream_synchronize(_sh(stream)))

    def download(self, count: int | None = None, dtype=np.float32,
                 stream: Stream | None = None) -> np.ndarray:
        itemsize = np.dtype(dtype).itemsize
        count = self.nbytes // itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        _check(lib().mcke_rt_memcpy_async(out.ctypes.data, self.ptr, out.nbytes, 1, _sh(stream)))
        _check(lib().mcke_rt_stream_synchronize(_sh(stream)))
        return out

    def memset(self, value: int = 0, stream: Stream | None = None) -> None:
        _check(lib().mcke_rt_memset_async(self.ptr, value, self.nbytes, _sh(stream)))

    def offset(self, nbytes: int) -> int:
        return self.ptr + nbytes

    def free(self) -> None:
        if self.ptr:
            lib().mcke_rt_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# Host data generators (the reference's fill_random map + a Box-Muller normal)
# ---------------------------------------------------------------------------
def fill_random(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().mcke_fill_random_f32(out.ctypes.data, n, seed, lo, hi)
    return out


def fill_normal(n: int, seed: int, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().mcke_fill_normal_f32(out.ctypes.data, n, seed, mu, sigma)
    return out


# ---------------------------------------------------------------------------
# Kernel launchers (kernels.hpp), returning Status
# ---------------------------------------------------------------------------
def launch_vector_add_f32(a, b, out, n: int, stream=None) -> Status:
    return _st(lib().mcke_launch_vector_add_f32(_ptr(a), _ptr(b), _ptr(out), n, _sh(stream)))


def launch_bias_act_f32(x, bias, y, rows: int, cols: int, act, vector_width: int,
                        stream=None, max_row_blocks: int = 0) -> Status:
    return _st(lib().mcke_launch_bias_act_f32(_ptr(x), _ptr(bias), _ptr(y), rows, cols,
                                              int(act), vector_width, _sh(stream),
                                              max_row_blocks))


def launch_bias_add_f32(x, bias, y, rows: int, cols: int, vector_width: int,
                        stream=None) -> Status:
    return _st(lib().mcke_launch_bias_add_f32(_ptr(x), _ptr(bias), _ptr(y), rows, cols,
                                              vector_width, _sh(stream)))


def launch_activation_f32(x, y, n: int, act, vector_width: int, stream=None) -> Status:
    return _st(lib().mcke_launch_activation_f32(_ptr(x), _ptr(y), n, int(act), vector_width,
                                                _sh(stream)))


def max_vector_width_f32(p, cols: int) -> int:
    return int(lib().mcke_max_vector_width_f32(_ptr(p), cols))


def row_reduce_workspace_bytes(rows: int, cols: int, variant) -> int:
    return int(lib().mcke_row_reduce_workspace_bytes(rows, cols, int(variant)))


def launch_row_reduce_f32(x, out, rows: int, cols: int, kind, variant, *rest) -> Status:
    """Both reference overloads: (..., stream) and (..., workspace, ws_bytes, stream)."""
    if len(rest) <= 1:
        stream = rest[0] if rest else None
        return _st(lib().mcke_launch_row_reduce_f32(_ptr(x), _ptr(out), rows, cols, int(kind),
                                                    int(variant), _sh(stream)))
    workspace, ws_bytes = rest[0], rest[1]
    stream = rest[2] if len(rest) > 2 else None
    return _st(lib().mcke_launch_row_reduce_ws_f32(_ptr(x), _ptr(out), rows, cols, int(kind),
                                                   int(variant), _ptr(workspace), ws_bytes,
                                                   _sh(stream)))


def launch_row_reduce_noalloc_f32(x, out, rows: int, cols: int, kind, stream=None) -> Status:
    """kTwoPass without a workspace and without allocating (no reference
    counterpart): the partials live in a per-GPU device array of the library."""
    return _st(lib().mcke_launch_row_reduce_noalloc_f32(_ptr(x), _ptr(out), rows, cols, int(kind),
                                                        _sh(stream)))


def launch_row_softmax_f32(x, y, rows: int, cols: int, variant, stream=None) -> Status:
    return _st(lib().mcke_launch_row_softmax_f32(_ptr(x), _ptr(y), rows, cols, int(variant),
                                                 _sh(stream)))


def launch_gemm_f32(a, b, c, m: int, n: int, k: int, alpha: float, beta: float, variant,
                    tile: GemmTile | None = None, stream=None) -> Status:
    tile = GemmTile() if tile is None else tile
    return _st(lib().mcke_launch_gemm_f32(_ptr(a), _ptr(b), _ptr(c), m, n, k, alpha, beta,
                                          int(variant), C.byref(tile), _sh(stream)))


def launch_gemm_bias_act_f32(a, b, bias, y, m: int, n: int, k: int, alpha: float, act,
                             tile: GemmTile | None = None, stream=None) -> Status:
    """y = act(alpha * A B + bias[col]) on kMfmaF32 with the bias and activation in
    the GEMM's epilogue: the bits of launch_gemm_f32 (beta = 0) followed by
    launch_bias_act_f32.  No reference counterpart (a fusion of its two launchers)."""
    tile = gemm_mfma_default_tile(m, n, k) if tile is None else tile
    return _st(lib().mcke_launch_gemm_bias_act_f32(_ptr(a), _ptr(b), _ptr(bias), _ptr(y), m, n,
                                                   k, alpha, int(act), C.byref(tile),
                                                   _sh(stream)))


def gemm_kernel_attrs(variant, tile: GemmTile | None = None):
    """Returns (Status, KernelAttrs)."""
    tile = GemmTile() if tile is None else tile
    out = KernelAttrs()
    st = _st(lib().mcke_gemm_kernel_attrs(int(variant), C.byref(tile), C.byref(out)))
    return st, out


def gemm_mfma_default_tile(m: int, n: int, k: int) -> GemmTile:
    t = GemmTile()
    _check(lib().mcke_gemm_mfma_default_tile(m, n, k, C.byref(t)))
    return t


def launch_gemm_lp(a, b, c, ab_dtype, c_dtype, m: int, n: int, k: int, alpha: float,
                   beta: float, tile: GemmTile | None = None, stream=None) -> Status:
    """16-bit-input GEMM (bf16 or fp16 A and B, fp32 accumulation, C in fp32 or
    the input type).  No reference counterpart: the reference reserves the
    kF16/kBF16 DType tags (dtype.hpp:33-41) but launches fp32 only."""
    tile = gemm_lp_default_tile(m, n, k) if tile is None else tile
    return _st(lib().mcke_launch_gemm_lp(_ptr(a), _ptr(b), _ptr(c), int(ab_dtype), int(c_dtype),
                                         m, n, k, alpha, beta, C.byref(tile), _sh(stream)))


def launch_gemm_lp_vendor(a, b, c, ab_dtype, c_dtype, m: int, n: int, k: int, alpha: float,
                          beta: float, stream=None) -> Status:
    """The vendor-library ceiling row of the 16-bit GEMM (rocBLAS gemm_ex)."""
    return _st(lib().mcke_launch_gemm_lp_vendor(_ptr(a), _ptr(b), _ptr(c), int(ab_dtype),
                                                int(c_dtype), m, n, k, alpha, beta, _sh(stream)))


def gemm_lp_kernel_attrs(ab_dtype, c_dtype, tile: GemmTile):
    """Returns (Status, KernelAttrs) of the whole-tile kernel."""
    out = KernelAttrs()
    st = _st(lib().mcke_gemm_lp_kernel_attrs(int(ab_dtype), int(c_dtype), C.byref(tile),
                                             C.byref(out)))
    return st, out


def gemm_lp_default_tile(m: int, n: int, k: int) -> GemmTile:
    t = GemmTile()
    _check(lib().mcke_gemm_lp_default_tile(m, n, k, C.byref(t)))
    return t


# ---------------------------------------------------------------------------
# Measured denominators (bench/fma_peak.cu, bench/stream_triad.cu counterparts)
# ---------------------------------------------------------------------------
def mfma_peak_flops(blocks: int, iters: int) -> int:
    return int(lib().mcke_mfma_peak_flops(blocks, iters))


def launch_mfma_peak_f32(seed, out, blocks: int, iters: int, stream=None) -> Status:
    return _st(lib().mcke_launch_mfma_peak_f32(_ptr(seed), _ptr(out), blocks, iters, _sh(stream)))


def launch_stream_copy_f32(x, y, n: int, stream=None) -> Status:
    return _st(lib().mcke_launch_stream_copy_f32(_ptr(x), _ptr(y), n, _sh(stream)))


def mfma_peak_lp_flops(blocks: int, iters: int) -> int:
    return int(lib().mcke_mfma_peak_lp_flops(blocks, iters))


def launch_mfma_peak_lp(ab_dtype, seed, out, blocks: int, iters: int, stream=None) -> Status:
    return _st(lib().mcke_launch_mfma_peak_lp(int(ab_dtype), _ptr(seed), _ptr(out), blocks, iters,
                                              _sh(stream)))


def mfma_clock_lp_flops(blocks: int, iters: int) -> int:
    return int(lib().mcke_mfma_clock_lp_flops(blocks, iters))


def launch_mfma_clock_lp(ab_dtype, shape: int, operand_bits, out, ticks, blocks: int, iters: int,
                         stream=None) -> Status:
    """Engine-clock probe for the 16-bit MFMA forms: shape 0 = 32x32x16, 1 = 16x16x32
    (see include/mcke_amd.h)."""
    return _st(lib().mcke_launch_mfma_clock_lp(int(ab_dtype), int(shape), _ptr(operand_bits),
                                               _ptr(out), _ptr(ticks), blocks, iters,
                                               _sh(stream)))


def launch_stream_triad_f32(b, c, a, scalar: float, n: int, stream=None) -> Status:
    return _st(lib().mcke_launch_stream_triad_f32(_ptr(b), _ptr(c), _ptr(a), scalar, n,
                                                  _sh(stream)))


LP_TILES = (                             # the 16-bit GEMM's instantiated tiles
    GemmTile(256, 256, 64, 16, 16),
    GemmTile(128, 128, 64, 8, 8),
    GemmTile(64, 64, 64, 4, 4),
)

MFMA_TILES = (
    GemmTile(256, 256, 32, 16, 16),
    GemmTile(256, 256, 16, 16, 16),
    GemmTile(128, 128, 32, 8, 8),
    GemmTile(128, 128, 16, 8, 8),
    GemmTile(64, 64, 32, 4, 4),
    GemmTile(32, 32, 32, 2, 2),
)
