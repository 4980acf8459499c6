"""MI355X runtime: ``ctypes`` over ``libamdhip64`` and ``libqutai_amd``.

Mirrors the reference CUDA runtime object (src/qutai/backends/cuda_runtime.py:81-363):
one process-wide ``Runtime`` bound to device 0, a stream-ordered size-class
pool allocator, synchronous host<->device copies, asynchronous kernel calls on
the default stream, error codes mapped to ``RuntimeError`` with the error
name, a sync-after-every-call debug switch and launch counters.  Instead of
compiling ``.cu`` text with NVRTC at first use (cuda_runtime.py:274-297), the
kernels are compiled ahead of time for gfx950 into ``libqutai_amd.so`` (built
by ``qutai_amd/build.py``) and called through its C ABI
(``include/qutai_amd.h``).  Importing ``qutai_amd`` never loads either
library; the first device touch does.
"""
from __future__ import annotations

import atexit
import ctypes
import os
import threading
from pathlib import Path

_runtime = None
_runtime_lock = threading.Lock()

LIBRARY = Path(__file__).resolve().parent.parent / "libqutai_amd.so"

# hipDeviceAttribute_t values of ROCm 7 (hip_runtime_api.h)
_ATTR_CC_MAJOR, _ATTR_CC_MINOR, _ATTR_CU_COUNT, _ATTR_CLOCK_KHZ = 23, 61, 63, 5
_MEMCPY_H2D, _MEMCPY_D2H, _MEMCPY_D2D = 1, 2, 3
_HIP_OOM = 2  # hipErrorOutOfMemory

QA_OK, QA_EINVAL, QA_EWORKSPACE, QA_ESCRATCH = 0, -1, -2, -3

_p, _i64, _i32, _f64, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.c_size_t

# C ABI of libqutai_amd (include/qutai_amd.h): name -> argument types.
SIGNATURES = {
    "qutai_amd_gemm": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                       _p, _sz, _p],
    "qutai_amd_gemm_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32],
    "qutai_amd_gemm_grouped": [_p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _p, _i64, _p],
    "qutai_amd_gemm_grouped_pair": [_p, _p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32,
                                    _p],
    "qutai_amd_gemm_swiglu": [_p, _p, _p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _i32, _p, _i64, _p],
    "qutai_amd_head_block_stats": [_p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p],
    "qutai_amd_head_block_loss": [_p, _p, _p, _p, _i64, _p],
    "qutai_amd_head_block_gradient": [_p, _p, _p, _p, _i64, _i64, _i64, _f64, _i32, _p],
    "qutai_amd_cast": [_p, _p, _i64, _i32, _i32, _p],
    "qutai_amd_fill": [_p, _i64, _f64, _i32, _p],
    "qutai_amd_add": [_p, _p, _p, _i64, _i32, _p],
    "qutai_amd_add_widen": [_p, _p, _p, _i64, _p],
    "qutai_amd_add_rows": [_p, _p, _p, _i64, _i64, _i32, _p],
    "qutai_amd_sum_middle": [_p, _p, _i64, _i64, _i64, _i32, _p],
    "qutai_amd_transpose_last2": [_p, _p, _i64, _i64, _i64, _i32, _p],
    "qutai_amd_swap_axes": [_p, _p, _i64, _i64, _i64, _i64, _i32, _p],
    "qutai_amd_softmax_rows": [_p, _p, _i64, _i64, _f64, _i32, _p],
    "qutai_amd_silu_mul": [_p, _p, _p, _i64, _i32, _p],
    "qutai_amd_silu_mul_backward": [_p, _p, _p, _p, _p, _i64, _i32, _p],
    "qutai_amd_route": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _sz, _p],
    "qutai_amd_route_workspace_size": [_i64, _i64, _i64],
    "qutai_amd_route_gather": [_p, _p, _p, _i64, _i64, _i32, _i32, _p],
    "qutai_amd_combine": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p],
    "qutai_amd_gemm_grouped_k": [_p, _p, _p, _p, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _p, _i64, _p],
    "qutai_amd_combine_backward": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "qutai_amd_route_backward": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "qutai_amd_scale": [_p, _p, _i64, _f64, _i32, _p],
    "qutai_amd_repitch": [_p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p],
    "qutai_amd_softmax_backward": [_p, _p, _p, _i64, _i64, _f64, _i32, _p],
    "qutai_amd_causal_mask": [_p, _p, _i64, _i64, _i64, _i64, _i32, _p],
    "qutai_amd_embedding": [_p, _p, _p, _i64, _i64, _i32, _p],
    "qutai_amd_embedding_backward": [_p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _p],
    "qutai_amd_rms_norm": [_p, _p, _p, _p, _i64, _i64, _f64, _i32, _p],
    "qutai_amd_rms_norm_bf16": [_p, _p, _p, _p, _p, _i64, _i64, _f64, _i32, _p],
    "qutai_amd_rms_norm_workspace": [_i64, _i64],
    "qutai_amd_rms_norm_backward": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p],
    "qutai_amd_silu": [_p, _p, _p, _i64, _i32, _i32, _p],
    "qutai_amd_rope": [_p, _p, _i64, _i64, _i64, _i64, _f64, _i64, _i32, _i32, _p],
    "qutai_amd_rope_rows": [_p, _p, _i64, _i64, _i64, _i64, _f64, _i64, _i32, _i64, _i64, _i32, _p],
    "qutai_amd_head_rows": [_p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p],
    "qutai_amd_head_loss": [_p, _p, _p, _i64, _i64, _i32, _p],
    "qutai_amd_head_gradient": [_p, _p, _p, _i64, _i64, _f64, _i32, _p],
    "qutai_amd_attention_fwd": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _f64, _i32, _p],
    "qutai_amd_attention_bwd": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _i64, _i64, _i64, _i64, _i64, _i32,
                                _i32, _f64, _i32, _p],
    "qutai_amd_attention_bwd_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i32],
    "qutai_amd_softmax": [_p, _p, _i64, _i64, _i64, _f64, _i32, _p],
    "qutai_amd_strided_copy": [_p, _p, _i32, _p, _p, _p, _i32, _p],
    "qutai_amd_binary": [_p, _p, _p, _i64, _i32, _i32, _p, _p],
    "qutai_amd_unary": [_p, _p, _p, _i64, _i32, _f64, _i32, _p, _p],
    "qutai_amd_reduce_sum": [_p, _p, _i64, _i64, _i64, _i32, _p, _sz, _p],
    "qutai_amd_reduce_sum_workspace_size": [_i64, _i64, _i64, _i32],
    "qutai_amd_gather": [_p, _p, _p, _i64, _i32, _p],
    "qutai_amd_scatter": [_p, _p, _p, _p, _i64, _i32, _p],
    "qutai_amd_device_arch": [_i32, ctypes.c_char_p, _sz],
    "qutai_amd_gemm_static": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32,
                              _i32, _p],
    "qutai_amd_gemm_static_capacity": [],
}
RESTYPES = {"qutai_amd_gemm_workspace_size": _sz, "qutai_amd_rms_norm_workspace": _i64,
            "qutai_amd_attention_bwd_workspace_size": _sz, "qutai_amd_reduce_sum_workspace_size": _sz,
            "qutai_amd_gemm_static_capacity": _sz, "qutai_amd_route_workspace_size": _sz}


def _hip_library():
    if ctypes.sizeof(ctypes.c_void_p) != 8:
        raise RuntimeError("the MI355X backend needs 64-bit Python")
    roots = [os.environ.get("ROCM_PATH"), os.environ.get("HIP_PATH"), "/opt/rocm"]
    candidates = [str(Path(root) / "lib" / "libamdhip64.so") for root in roots if root]
    candidates.append("libamdhip64.so")
    errors = []
    for candidate in candidates:
        try:
            return ctypes.CDLL(candidate, mode=ctypes.RTLD_GLOBAL)
        except OSError as error:
            errors.append(str(error))
    raise RuntimeError("libamdhip64 not found: " + "; ".join(errors))


def load_library(path: Path = LIBRARY):
    """Load libqutai_amd and bind its C ABI (no device touched)."""
    if not path.exists():
        raise RuntimeError(f"{path.name} is not built; run `python -m qutai_amd.build` (hipcc, gfx950)")
    library = ctypes.CDLL(str(path))
    for name, arguments in SIGNATURES.items():
        function = getattr(library, name)
        function.argtypes = arguments
        function.restype = RESTYPES.get(name, ctypes.c_int)
    return library


class Runtime:
    """Device 0, default stream; calls are queued asynchronously, reads synchronise."""

    def __init__(self):
        self._lock = threading.RLock()
        self._allocations = {}
        self._blocks = {}
        self._available = {}
        self.allocated_bytes = self.reserved_bytes = 0
        self.peak_allocated_bytes = self.peak_reserved_bytes = 0
        self.cache_limit_bytes = 1 << 30
        self.launches = 0
        self.mfma_launches = 0
        self.debug_sync = os.environ.get("QUTAI_AMD_SYNC") == "1"
        self._closed = False
        # pinned staging ring for asynchronous host-to-device uploads
        self._staging, self._staging_at, self._staging_pending = None, 0, []
        self.hip = _hip_library()
        self._bind_hip()
        self.lib = load_library()
        self._check(self._init(0), "hipInit")
        count = ctypes.c_int()
        self._check(self._device_count(ctypes.byref(count)), "hipGetDeviceCount")
        if count.value < 1:
            raise RuntimeError("no AMD GPU visible")
        self.device = 0
        self._check(self._set_device(self.device), "hipSetDevice")
        name = ctypes.create_string_buffer(256)
        self._check(self._device_name(name, len(name), self.device), "hipDeviceGetName")
        self.name = name.value.decode("utf8", "replace")
        arch = ctypes.create_string_buffer(256)
        self._check(self.lib.qutai_amd_device_arch(self.device, arch, len(arch)), "hipGetDeviceProperties")
        self.arch = arch.value.decode("ascii", "replace")
        self.compute_capability = (self._attribute(_ATTR_CC_MAJOR), self._attribute(_ATTR_CC_MINOR))
        self.cu_count = self._attribute(_ATTR_CU_COUNT)
        self.clock_khz = self._attribute(_ATTR_CLOCK_KHZ)
        if not self.arch.startswith("gfx950"):
            raise RuntimeError(f"libqutai_amd is built for gfx950 only; device 0 is {self.arch or 'unknown'}")
        version = ctypes.c_int()
        self._check(self._driver_version(ctypes.byref(version)), "hipDriverGetVersion")
        self.driver_version = version.value
        free, total = ctypes.c_size_t(), ctypes.c_size_t()
        self._check(self._mem_info(ctypes.byref(free), ctypes.byref(total)), "hipMemGetInfo")
        self.total_memory = total.value
        # Idle-cache cap: the reference keeps 1 GiB (a WDDM budget,
        # cuda_runtime.py:214-216); with 288 GB of HBM a decoder step's
        # transient buffers exceed that, and every overflow drains the device
        # and frees the whole cache, so the cap is 1/16 of the device here.
        self.cache_limit_bytes = max(1 << 30, self.total_memory // 16)
        atexit.register(self.close)

    # ---- binding -------------------------------------------------------------
    def _bind_hip(self):
        h = self.hip

        def bind(name, arguments, result=ctypes.c_int):
            function = getattr(h, name)
            function.argtypes = arguments
            function.restype = result
            return function

        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        self._init = bind("hipInit", [ctypes.c_uint])
        self._device_count = bind("hipGetDeviceCount", [ctypes.POINTER(ctypes.c_int)])
        self._set_device = bind("hipSetDevice", [ctypes.c_int])
        self._device_name = bind("hipDeviceGetName", [ctypes.c_char_p, ctypes.c_int, ctypes.c_int])
        self._device_attribute = bind("hipDeviceGetAttribute", [ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                                                ctypes.c_int])
        self._driver_version = bind("hipDriverGetVersion", [ctypes.POINTER(ctypes.c_int)])
        self._sync = bind("hipDeviceSynchronize", [])
        self._mem_info = bind("hipMemGetInfo", [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)])
        self._malloc = bind("hipMalloc", [ctypes.POINTER(ctypes.c_void_p), sz])
        self._free = bind("hipFree", [vp])
        self._memcpy = bind("hipMemcpy", [vp, vp, sz, ctypes.c_int])
        self._memcpy_async = bind("hipMemcpyAsync", [vp, vp, sz, ctypes.c_int, vp])
        self._host_malloc = bind("hipHostMalloc", [ctypes.POINTER(ctypes.c_void_p), sz, ctypes.c_uint])
        self._host_free = bind("hipHostFree", [vp])
        self._event_create_flags = bind("hipEventCreateWithFlags", [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint])
        self._event_create = bind("hipEventCreate", [ctypes.POINTER(ctypes.c_void_p)])
        self._event_record = bind("hipEventRecord", [vp, vp])
        self._event_sync = bind("hipEventSynchronize", [vp])
        self._event_elapsed = bind("hipEventElapsedTime", [ctypes.POINTER(ctypes.c_float), vp, vp])
        self._event_destroy = bind("hipEventDestroy", [vp])
        self._error_name = bind("hipGetErrorName", [ctypes.c_int], ctypes.c_char_p)
        self._error_string = bind("hipGetErrorString", [ctypes.c_int], ctypes.c_char_p)

    def _attribute(self, attribute):
        value = ctypes.c_int()
        self._check(self._device_attribute(ctypes.byref(value), attribute, self.device), "hipDeviceGetAttribute")
        return value.value

    def _check(self, result, operation):
        if result:
            name = (self._error_name(result) or str(result).encode()).decode("utf8", "replace")
            detail = (self._error_string(result) or b"").decode("utf8", "replace")
            raise RuntimeError(f"HIP {operation} failed: {name} ({detail})")

    def _current(self):
        if self._closed:
            raise RuntimeError("the MI355X runtime is closed")

    # ---- memory (pool semantics of cuda_runtime.py:184-228) ------------------
    def allocate(self, nbytes: int) -> int:
        if nbytes < 0:
            raise ValueError("byte count must be non-negative")
        if not nbytes:
            return 0
        unit = 65536 if nbytes >= 65536 else 512
        capacity = ((nbytes + unit - 1) // unit) * unit
        with self._lock:
            self._current()
            pool = self._available.get(capacity, [])
            if pool:
                pointer = pool.pop()
            else:
                value = ctypes.c_void_p()
                status = self._malloc(ctypes.byref(value), capacity)
                if status == _HIP_OOM:  # release the idle cache, then retry once
                    self.empty_cache()
                    status = self._malloc(ctypes.byref(value), capacity)
                self._check(status, "hipMalloc")
                pointer = value.value
                self._blocks[pointer] = capacity
                self.reserved_bytes += capacity
                self.peak_reserved_bytes = max(self.peak_reserved_bytes, self.reserved_bytes)
            self._allocations[pointer] = nbytes
            self.allocated_bytes += nbytes
            self.peak_allocated_bytes = max(self.peak_allocated_bytes, self.allocated_bytes)
            return pointer

    def free(self, ptr: int):
        with self._lock:
            if self._closed or ptr not in self._allocations:
                return
            self.allocated_bytes -= self._allocations.pop(ptr)
            # every later use is on the same default stream, so reuse is ordered
            self._available.setdefault(self._blocks[ptr], []).append(ptr)
            if self.reserved_bytes - self.allocated_bytes > self.cache_limit_bytes:
                self.empty_cache()

    def empty_cache(self):
        with self._lock:
            self._current()
            self._check(self._sync(), "hipDeviceSynchronize")
            for pointers in self._available.values():
                for ptr in pointers:
                    self._check(self._free(ptr), "hipFree")
                    self.reserved_bytes -= self._blocks.pop(ptr)
            self._available.clear()

    def memory_stats(self):
        return {"allocated_bytes": self.allocated_bytes, "reserved_bytes": self.reserved_bytes,
                "peak_allocated_bytes": self.peak_allocated_bytes, "peak_reserved_bytes": self.peak_reserved_bytes}

    def reset_peak_memory_stats(self):
        self.peak_allocated_bytes = self.allocated_bytes
        self.peak_reserved_bytes = self.reserved_bytes

    # ---- copies -----------------------------------------------------------------
    @staticmethod
    def _host_buffer(buffer):
        view = memoryview(buffer)
        if view.readonly or not view.c_contiguous:
            raise ValueError("host buffer must be contiguous and writable")
        return (ctypes.c_ubyte * view.nbytes).from_buffer(buffer), view.nbytes

    STAGING_BYTES = 16 << 20  # pinned ring; uploads up to a quarter of it are asynchronous

    def upload(self, ptr: int, buffer):
        """Host bytes into device memory, in order with the kernels of the
        default stream.  Small uploads are copied into a pinned staging ring
        and sent with hipMemcpyAsync, so the host does not wait for the kernels
        queued before them; an event per upload guards its ring region until
        the copy has run.  Larger ones use a synchronous hipMemcpy."""
        host, nbytes = self._host_buffer(buffer)
        with self._lock:
            self._current()
            if not nbytes:
                return
            if nbytes > self.STAGING_BYTES // 4:
                self._check(self._memcpy(ptr, host, nbytes, _MEMCPY_H2D), "hipMemcpy HtoD")
                return
            if self._staging is None:
                value = ctypes.c_void_p()
                self._check(self._host_malloc(ctypes.byref(value), self.STAGING_BYTES, 0), "hipHostMalloc")
                self._staging = value.value
            start = self._staging_at if self._staging_at + nbytes <= self.STAGING_BYTES else 0
            end = start + nbytes
            # wait for the copies that still read the region about to be overwritten
            keep = []
            for lo, hi, event in self._staging_pending:
                if lo < end and start < hi:
                    self._check(self._event_sync(event), "hipEventSynchronize")
                    self._event_destroy(event)
                else:
                    keep.append((lo, hi, event))
            ctypes.memmove(self._staging + start, host, nbytes)
            self._check(self._memcpy_async(ptr, self._staging + start, nbytes, _MEMCPY_H2D, None),
                        "hipMemcpyAsync HtoD")
            event = ctypes.c_void_p()
            self._check(self._event_create_flags(ctypes.byref(event), 2), "hipEventCreateWithFlags")  # no timing
            self._check(self._event_record(event, None), "hipEventRecord")
            keep.append((start, end, event.value))
            self._staging_pending = keep
            self._staging_at = (end + 255) // 256 * 256

    def download(self, ptr: int, buffer):
        host, nbytes = self._host_buffer(buffer)
        with self._lock:
            self._current()
            if nbytes:
                self._check(self._sync(), "hipDeviceSynchronize")
                self._check(self._memcpy(host, ptr, nbytes, _MEMCPY_D2H), "hipMemcpy DtoH")

    def copy(self, dst: int, src: int, nbytes: int):
        if nbytes < 0:
            raise ValueError("byte count must be non-negative")
        with self._lock:
            self._current()
            if nbytes:
                self._check(self._memcpy_async(dst, src, nbytes, _MEMCPY_D2D, None), "hipMemcpyAsync DtoD")

    def synchronize(self):
        with self._lock:
            self._current()
            self._check(self._sync(), "hipDeviceSynchronize")

    # ---- kernels ---------------------------------------------------------------
    def call(self, name: str, *arguments, mfma: bool = False):
        """Run one libqutai_amd entry point on the default stream."""
        with self._lock:
            self._current()
            status = getattr(self.lib, name)(*arguments, None)
            if status == QA_EINVAL:
                raise ValueError(f"{name}: arguments rejected by libqutai_amd")
            if status == QA_EWORKSPACE:
                raise RuntimeError(f"{name}: workspace missing or too small")
            if status == QA_ESCRATCH:
                raise RuntimeError(f"{name}: the operands need more workspace than the fixed "
                                   f"{self.lib.qutai_amd_gemm_static_capacity() >> 20} MiB device scratch")
            self._check(status, name)
            self.launches += 1
            if mfma:
                self.mfma_launches += 1
            if self.debug_sync:
                self._check(self._sync(), f"hipDeviceSynchronize after {name}")

    # ---- events (timing on the default stream) ---------------------------------
    def event(self):
        value = ctypes.c_void_p()
        self._check(self._event_create(ctypes.byref(value)), "hipEventCreate")
        return value.value

    def record(self, event):
        self._check(self._event_record(event, None), "hipEventRecord")

    def elapsed_ms(self, start, end):
        self._check(self._event_sync(end), "hipEventSynchronize")
        value = ctypes.c_float()
        self._check(self._event_elapsed(ctypes.byref(value), start, end), "hipEventElapsedTime")
        return value.value

    def destroy_event(self, event):
        self._event_destroy(event)

    def close(self):
        with self._lock:
            if self._closed:
                return
            self._closed = True
            self._sync()
            for _, _, event in self._staging_pending:
                self._event_destroy(event)
            self._staging_pending = []
            if self._staging is not None:
                self._host_free(self._staging)
                self._staging = None
            for pointer in self._blocks:
                self._free(pointer)
            self._allocations.clear()
            self._blocks.clear()
            self._available.clear()
            self.allocated_bytes = self.reserved_bytes = 0


def get_runtime() -> Runtime:
    """First device touch loads the libraries and binds device 0."""
    global _runtime
    with _runtime_lock:
        if _runtime is None or _runtime._closed:
            _runtime = Runtime()
        return _runtime
