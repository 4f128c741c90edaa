"""Python binding of the MI355X flash-attention C ABI (``include/notcute_flash.h``).

This is a ctypes mirror of the reference's public ``flash`` / ``cuda`` / ``benchmark`` modules
(src/flash.zig, src/cuda.zig, src/benchmark.zig) over ``libnotcute_flash.so``. It holds no compute:
every launch goes to the gfx950 kernels in the embedded code object, and loading fails loudly when
the library has not been built.

Errors surface as :class:`NcError`, whose ``name`` is the reference's ``CudaError`` member
(src/cuda.zig:134-151), e.g. ``InvalidValue`` for a rejected ``Options`` (src/flash.zig:16-28).
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# NC_LIBRARY selects another build of the same library (e.g. the host-sanitizer build of
# `make host-sanitize`); by default the in-tree one.
LIB_PATH = os.environ.get("NC_LIBRARY") or os.path.join(HERE, "libnotcute_flash.so")

STATUS_NAMES = [
    "Success", "OutOfMemory", "Overflow", "SharedObjectInitFailed", "NotFound", "InvalidValue",
    "InvalidContext", "InvalidDevice", "InvalidImage", "ContextIsDestroyed", "LaunchFailed",
    "LaunchOutOfResources", "LaunchTimeout", "IllegalAddress", "NoDevice", "NotInitialized",
    "UnknownError",
]


class NcError(RuntimeError):
    """A non-zero nc_status; ``name`` is the matching CudaError name of src/cuda.zig:134-151."""

    def __init__(self, status: int, what: str = "", detail: str = ""):
        self.status = int(status)
        self.name = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else "UnknownError"
        msg = f"{what}: {self.name} ({self.status})"
        if detail:
            msg += f" [{detail}]"
        super().__init__(msg)


# element_type values (NC_ELEMENT_F16 / NC_ELEMENT_BF16).
ELEMENT_TYPES = {"f16": 0, "bf16": 1}


class FlashOptions(ctypes.Structure):
    """flash.Options (src/flash.zig:5-14) + optional row strides (0 = head_dim)."""

    _fields_ = [
        ("batch_heads", ctypes.c_uint64),
        ("seq_len", ctypes.c_uint64),
        ("head_dim", ctypes.c_uint64),
        ("q_stride", ctypes.c_uint64),
        ("k_stride", ctypes.c_uint64),
        ("v_stride", ctypes.c_uint64),
        ("o_stride", ctypes.c_uint64),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_uint32),
        ("q_row_stride", ctypes.c_uint64),
        ("k_row_stride", ctypes.c_uint64),
        ("v_row_stride", ctypes.c_uint64),
        ("o_row_stride", ctypes.c_uint64),
        ("element_type", ctypes.c_uint32),
    ]


class KernelSelection(ctypes.Structure):
    """flash.KernelSelection (src/flash.zig:72-76) + launch geometry."""

    _fields_ = [
        ("name", ctypes.c_char_p),
        ("label", ctypes.c_char_p),
        ("reference_name", ctypes.c_char_p),
        ("threads", ctypes.c_uint32),
        ("grid", ctypes.c_uint32 * 3),
        ("block_m", ctypes.c_uint32),
        ("block_n", ctypes.c_uint32),
        ("kv_splits", ctypes.c_uint32),
        ("lds_bytes", ctypes.c_uint32),
        ("aligned", ctypes.c_uint32),
        ("scratch_bytes", ctypes.c_uint64),
    ]


class KernelArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("seq_len", ctypes.c_uint64),
        ("head_dim", ctypes.c_uint64),
        ("q_stride", ctypes.c_uint64),
        ("k_stride", ctypes.c_uint64),
        ("v_stride", ctypes.c_uint64),
        ("o_stride", ctypes.c_uint64),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_uint32),
        ("q_row_stride", ctypes.c_uint64),
        ("k_row_stride", ctypes.c_uint64),
        ("v_row_stride", ctypes.c_uint64),
        ("o_row_stride", ctypes.c_uint64),
        ("batch_heads", ctypes.c_uint32),
        ("num_q_blocks", ctypes.c_uint32),
        ("scratch", ctypes.c_void_p),
        ("balance_tail", ctypes.c_uint32),
    ]


class LaunchConfig(ctypes.Structure):
    """LaunchConfig + Dim3 (src/cuda.zig:344-356)."""

    _fields_ = [
        ("grid", ctypes.c_uint32 * 3),
        ("block", ctypes.c_uint32 * 3),
        ("shared_mem_bytes", ctypes.c_uint32),
        ("stream", ctypes.c_void_p),
    ]


class FunctionAttributes(ctypes.Structure):
    """Function.Attributes (src/cuda.zig:362-388)."""

    _fields_ = [
        ("max_threads_per_block", ctypes.c_int32),
        ("shared_size_bytes", ctypes.c_int32),
        ("const_size_bytes", ctypes.c_int32),
        ("local_size_bytes", ctypes.c_int32),
        ("num_regs", ctypes.c_int32),
        ("ptx_version", ctypes.c_int32),
        ("binary_version", ctypes.c_int32),
    ]


class DeviceAttributes(ctypes.Structure):
    """cuda.OccupancyCalculator fields (src/cuda.zig:228-245) plus the gfx950 LDS/clock/name."""

    _fields_ = [
        ("max_threads_per_block", ctypes.c_int32),
        ("max_shared_memory_per_block", ctypes.c_int32),
        ("max_registers_per_sm", ctypes.c_int32),
        ("max_threads_per_sm", ctypes.c_int32),
        ("sm_count", ctypes.c_int32),
        ("warp_size", ctypes.c_int32),
        ("max_shared_memory_per_sm", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("name", ctypes.c_char * 64),
    ]


class FlashWork(ctypes.Structure):
    _fields_ = [
        ("flops_reference", ctypes.c_uint64),
        ("flops_halfsquare", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
    ]


class BenchmarkOptions(ctypes.Structure):
    """BenchmarkOptions (src/benchmark.zig:26-32)."""

    _fields_ = [
        ("warmup_iters", ctypes.c_uint32),
        ("iters", ctypes.c_uint32),
        ("bytes_processed", ctypes.c_uint64),
        ("flops_processed", ctypes.c_uint64),
        ("stream", ctypes.c_void_p),
    ]


class BenchmarkResult(ctypes.Structure):
    """BenchmarkResult (src/benchmark.zig:6-11)."""

    _fields_ = [
        ("mean_ms", ctypes.c_float),
        ("min_ms", ctypes.c_float),
        ("max_ms", ctypes.c_float),
        ("throughput_gbps", ctypes.c_float),
        ("tflops", ctypes.c_float),
        ("has_gbps", ctypes.c_uint32),
        ("has_tflops", ctypes.c_uint32),
    ]


_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_SIGS = {
    "nc_status_name": (ctypes.c_char_p, [ctypes.c_int]),
    "nc_last_error_string": (ctypes.c_char_p, []),
    "nc_status_from_hip": (ctypes.c_int, [ctypes.c_int]),
    "nc_version": (ctypes.c_char_p, []),
    "nc_init": (ctypes.c_int, []),
    "nc_deinit": (None, []),
    "nc_device_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "nc_device_synchronize": (ctypes.c_int, []),
    "nc_malloc": (ctypes.c_int, [ctypes.POINTER(_P), ctypes.c_size_t]),
    "nc_free": (None, [_P]),
    "nc_memcpy_htod": (ctypes.c_int, [_P, _P, ctypes.c_size_t]),
    "nc_memcpy_dtoh": (ctypes.c_int, [_P, _P, ctypes.c_size_t]),
    "nc_memset": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_size_t]),
    "nc_module_load_data": (ctypes.c_int, [ctypes.POINTER(_P), _P]),
    "nc_module_load_file": (ctypes.c_int, [ctypes.POINTER(_P), ctypes.c_char_p]),
    "nc_module_load_embedded": (ctypes.c_int, [ctypes.POINTER(_P)]),
    "nc_module_unload": (ctypes.c_int, [_P]),
    "nc_module_get_function": (ctypes.c_int, [ctypes.POINTER(_P), _P, ctypes.c_char_p]),
    "nc_function_launch": (ctypes.c_int, [_P, ctypes.POINTER(LaunchConfig), ctypes.POINTER(_P)]),
    "nc_function_get_attributes": (ctypes.c_int, [_P, ctypes.POINTER(FunctionAttributes)]),
    "nc_device_get_attributes": (ctypes.c_int, [ctypes.POINTER(DeviceAttributes)]),
    "nc_function_max_active_blocks": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int)]),
    "nc_stream_create": (ctypes.c_int, [ctypes.POINTER(_P)]),
    "nc_stream_destroy": (ctypes.c_int, [_P]),
    "nc_stream_synchronize": (ctypes.c_int, [_P]),
    "nc_event_create": (ctypes.c_int, [ctypes.POINTER(_P)]),
    "nc_event_create_timing": (ctypes.c_int, [ctypes.POINTER(_P)]),
    "nc_event_destroy": (ctypes.c_int, [_P]),
    "nc_event_record": (ctypes.c_int, [_P, _P]),
    "nc_event_record_node": (ctypes.c_int, [_P, _P]),
    "nc_event_synchronize": (ctypes.c_int, [_P]),
    "nc_event_elapsed": (ctypes.c_int, [ctypes.POINTER(ctypes.c_float), _P, _P]),
    "nc_stream_begin_capture": (ctypes.c_int, [_P]),
    "nc_stream_end_capture": (ctypes.c_int, [_P, ctypes.POINTER(_P)]),
    "nc_graph_launch": (ctypes.c_int, [_P, _P]),
    "nc_graph_destroy": (ctypes.c_int, [_P]),
    "nc_flash_options_init": (None, [ctypes.POINTER(FlashOptions)]),
    "nc_flash_validate": (ctypes.c_int, [ctypes.POINTER(FlashOptions)]),
    "nc_flash_select_kernel": (ctypes.c_int, [ctypes.POINTER(FlashOptions), ctypes.POINTER(KernelSelection)]),
    "nc_flash_select_kernel_for": (
        ctypes.c_int, [ctypes.POINTER(FlashOptions), _P, _P, _P, _P, ctypes.POINTER(KernelSelection)]),
    "nc_flash_kernel_params": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_void_p, ctypes.POINTER(_P), ctypes.c_uint32,
                                              ctypes.POINTER(ctypes.c_uint32)]),
    "nc_flash_pack_args": (
        ctypes.c_int,
        [ctypes.POINTER(FlashOptions), ctypes.POINTER(KernelSelection), _P, _P, _P, _P, ctypes.POINTER(KernelArgs)]),
    "nc_flash_launch": (
        ctypes.c_int,
        [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, ctypes.c_size_t,
         ctypes.POINTER(FlashOptions)]),
    "nc_flash_launch_async": (
        ctypes.c_int,
        [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, ctypes.c_size_t,
         ctypes.POINTER(FlashOptions), _P]),
    "nc_flash_work_model": (ctypes.c_int, [ctypes.POINTER(FlashOptions), ctypes.POINTER(FlashWork)]),
    "nc_flash_launch_noalloc": (
        ctypes.c_int,
        [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, ctypes.c_size_t,
         ctypes.POINTER(FlashOptions), _P]),
    "nc_flash_reserve_workspace": (ctypes.c_int, [_P, ctypes.POINTER(FlashOptions), ctypes.POINTER(_P)]),
    "nc_flash_reset_scratch": (ctypes.c_int, [_P]),
    "nc_flash_kernel_scratch_bytes": (
        ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(FlashOptions), ctypes.POINTER(_U64)]),
    "nc_benchmark_options_init": (None, [ctypes.POINTER(BenchmarkOptions)]),
    "nc_benchmark_run_kernel": (
        ctypes.c_int,
        [ctypes.POINTER(BenchmarkOptions), _P, ctypes.POINTER(LaunchConfig), ctypes.POINTER(_P),
         ctypes.POINTER(BenchmarkResult)]),
    "nc_benchmark_finish": (
        None, [ctypes.POINTER(ctypes.c_float), ctypes.c_uint32, _U64, _U64, ctypes.POINTER(BenchmarkResult)]),
    "nc_fill_flash_input": (None, [_P, ctypes.c_size_t, _U64, _U64, ctypes.c_float]),
    "nc_fill_uniform_f16": (None, [_P, ctypes.c_size_t, _U64, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]),
    "nc_fill_normal_f16": (None, [_P, ctypes.c_size_t, _U64, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]),
    "nc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "nc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "nc_fill_uniform_bf16": (None, [_P, ctypes.c_size_t, _U64, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]),
    "nc_fill_normal_bf16": (None, [_P, ctypes.c_size_t, _U64, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]),
    "nc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
    "nc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
}

_lib: Optional[ctypes.CDLL] = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libnotcute_flash.so; raises if it is missing (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is not built: run `make -C not-cute-zig_amd` or __graft_entry__.build() first")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def lib() -> ctypes.CDLL:
    return load_library()


def check(status: int, what: str) -> None:
    if status != 0:
        detail = (lib().nc_last_error_string() or b"").decode(errors="replace")
        raise NcError(status, what, detail)


# ---------------------------------------------------------------------------------------------
# flash module
# ---------------------------------------------------------------------------------------------

def options(*, seq_len: int, head_dim: int, q_stride: Optional[int] = None, k_stride: Optional[int] = None,
            v_stride: Optional[int] = None, o_stride: Optional[int] = None, scale: Optional[float] = None,
            batch_heads: int = 1, causal: bool = False, q_row_stride: int = 0, k_row_stride: int = 0,
            v_row_stride: int = 0, o_row_stride: int = 0, dtype: str = "f16") -> FlashOptions:
    """Build flash.Options; unspecified slice strides default to the dense seq_len*head_dim and an
    unspecified scale to 1/sqrt(head_dim) (the reference's callers, src/main.zig:225, 983).
    dtype "f16" (the reference's) or "bf16" sets element_type."""
    o = FlashOptions()
    lib().nc_flash_options_init(ctypes.byref(o))
    dense = seq_len * head_dim
    o.batch_heads = batch_heads
    o.seq_len = seq_len
    o.head_dim = head_dim
    o.q_stride = dense if q_stride is None else q_stride
    o.k_stride = dense if k_stride is None else k_stride
    o.v_stride = dense if v_stride is None else v_stride
    o.o_stride = dense if o_stride is None else o_stride
    o.scale = (1.0 / float(np.sqrt(head_dim))) if scale is None else scale
    o.causal = 1 if causal else 0
    o.q_row_stride = q_row_stride
    o.k_row_stride = k_row_stride
    o.v_row_stride = v_row_stride
    o.o_row_stride = o_row_stride
    o.element_type = ELEMENT_TYPES[dtype]
    return o


def validate(opts: FlashOptions) -> None:
    check(lib().nc_flash_validate(ctypes.byref(opts)), "flash.validate")


def select_kernel(opts: FlashOptions) -> KernelSelection:
    sel = KernelSelection()
    check(lib().nc_flash_select_kernel(ctypes.byref(opts), ctypes.byref(sel)), "flash.selectKernel")
    return sel


def select_kernel_for(opts: FlashOptions, q: int, k: int, v: int, o: int) -> KernelSelection:
    sel = KernelSelection()
    check(lib().nc_flash_select_kernel_for(ctypes.byref(opts), q, k, v, o, ctypes.byref(sel)),
          "flash.selectKernel")
    return sel


def work_model(opts: FlashOptions) -> FlashWork:
    w = FlashWork()
    check(lib().nc_flash_work_model(ctypes.byref(opts), ctypes.byref(w)), "flash.workModel")
    return w


def pack_args(opts: FlashOptions, sel: KernelSelection, q: int, k: int, v: int, o: int,
              module: Optional["Module"] = None) -> KernelArgs:
    """The kernel argument block for `sel`. A kernel that needs scratch memory (sel.scratch_bytes > 0)
    gets `module`'s workspace, reserved here; without a module such a selection is refused."""
    a = KernelArgs()
    check(lib().nc_flash_pack_args(ctypes.byref(opts), ctypes.byref(sel), q, k, v, o, ctypes.byref(a)),
          "flash.packArgs")
    if sel.scratch_bytes:
        if module is None:
            raise ValueError(f"{sel.name.decode()} needs {sel.scratch_bytes} bytes of scratch: pass the module")
        a.scratch = reserve_workspace(module, opts)
    return a


MAX_KERNEL_PARAMS = 20  # NC_FLASH_MAX_KERNEL_PARAMS


def kernel_params(name: str, args: KernelArgs) -> list:
    """nc_flash_kernel_params as ctypes objects for Function.launch and run_kernel: [args] for a kernel
    that takes the argument block as one parameter, else (the dense-layout `q1s8p1d`/`q1s8p2d` kernels) one
    object per field,
    each aliasing that field of `args`."""
    arr = (_P * MAX_KERNEL_PARAMS)()
    n = ctypes.c_uint32()
    check(lib().nc_flash_kernel_params(name.encode(), ctypes.byref(args), arr, MAX_KERNEL_PARAMS, ctypes.byref(n)),
          f"flash.kernelParams({name})")
    if n.value == 1:
        return [args]
    base = ctypes.addressof(args)
    views = []
    for i, (fname, ftype) in enumerate(KernelArgs._fields_):
        off = getattr(KernelArgs, fname).offset
        if arr[i] != base + off:
            raise RuntimeError(f"kernel_params({name}): parameter {i} is not field {fname}")
        views.append(ftype.from_buffer(args, off))
    return views


def kernel_scratch_bytes(name: str, opts: FlashOptions) -> int:
    """nc_flash_kernel_scratch_bytes: scratch the named kernel needs for `opts` (0 for most)."""
    n = ctypes.c_uint64()
    check(lib().nc_flash_kernel_scratch_bytes(name.encode(), ctypes.byref(opts), ctypes.byref(n)),
          "flash.kernelScratchBytes")
    return int(n.value)


def reserve_workspace(module: "Module", opts: FlashOptions) -> Optional[int]:
    """nc_flash_reserve_workspace: the module's workspace sized for `opts` (None when not needed)."""
    p = ctypes.c_void_p()
    check(lib().nc_flash_reserve_workspace(module.handle, ctypes.byref(opts), ctypes.byref(p)),
          "flash.reserveWorkspace")
    return p.value


def reset_scratch(module: Optional["Module"] = None) -> None:
    """nc_flash_reset_scratch: zero the pair-split exchange counters (static scratch of the current
    GPU, and `module`'s workspaces) and synchronise; no launch may be in flight."""
    check(lib().nc_flash_reset_scratch(module.handle if module is not None else None), "flash.resetScratch")


# ---------------------------------------------------------------------------------------------
# device, memory, module, stream, event
# ---------------------------------------------------------------------------------------------

def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib().nc_device_count(ctypes.byref(n)), "deviceCount")
    return n.value


def init() -> None:
    check(lib().nc_init(), "cuda.init")


def synchronize() -> None:
    check(lib().nc_device_synchronize(), "deviceSynchronize")


class DeviceBuffer:
    """A device allocation (cuda.malloc / free, src/cuda.zig:259-276)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().nc_malloc(ctypes.byref(p), max(self.nbytes, 1)), "cuda.malloc")
        self.ptr = int(p.value)

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset_bytes: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset_bytes + arr.nbytes > self.nbytes:
            raise NcError(5, "cuda.memcpy")
        check(lib().nc_memcpy_htod(self.ptr + offset_bytes, arr.ctypes.data, arr.nbytes), "cuda.memcpy")

    def download(self, dtype, count: int, offset_bytes: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if offset_bytes + out.nbytes > self.nbytes:
            raise NcError(5, "cuda.memcpy")
        check(lib().nc_memcpy_dtoh(out.ctypes.data, self.ptr + offset_bytes, out.nbytes), "cuda.memcpy")
        return out

    def memset(self, byte_value: int) -> None:
        check(lib().nc_memset(self.ptr, byte_value, self.nbytes), "memset")

    def free(self) -> None:
        if self.ptr:
            lib().nc_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Function:
    def __init__(self, handle: int, name: str):
        self.handle = handle
        self.name = name

    def attributes(self) -> FunctionAttributes:
        a = FunctionAttributes()
        check(lib().nc_function_get_attributes(self.handle, ctypes.byref(a)), "Function.getAttributes")
        return a

    def max_active_blocks(self, block_threads: int, dynamic_shared_bytes: int = 0) -> int:
        """Workgroups of `block_threads` threads resident on one CU at once."""
        n = ctypes.c_int(0)
        check(lib().nc_function_max_active_blocks(self.handle, block_threads, dynamic_shared_bytes, ctypes.byref(n)),
              f"occupancy({self.name})")
        return n.value

    def launch(self, grid: Sequence[int], block: Sequence[int], params: Sequence[ctypes._SimpleCData],
               stream: Optional[int] = None, shared_mem_bytes: int = 0) -> None:
        cfg = make_config(grid, block, stream, shared_mem_bytes)
        arr = (ctypes.c_void_p * len(params))(*[ctypes.cast(ctypes.pointer(p), ctypes.c_void_p) for p in params])
        check(lib().nc_function_launch(self.handle, ctypes.byref(cfg), arr), f"Function.launch({self.name})")


def device_attributes() -> DeviceAttributes:
    """cuda.getDevice + OccupancyCalculator.init (src/cuda.zig:228-245) for device 0."""
    a = DeviceAttributes()
    check(lib().nc_device_get_attributes(ctypes.byref(a)), "device attributes")
    return a


def make_config(grid: Sequence[int], block: Sequence[int], stream: Optional[int] = None,
                shared_mem_bytes: int = 0) -> LaunchConfig:
    cfg = LaunchConfig()
    g = list(grid) + [1] * (3 - len(grid))
    b = list(block) + [1] * (3 - len(block))
    for i in range(3):
        cfg.grid[i] = g[i]
        cfg.block[i] = b[i]
    cfg.shared_mem_bytes = shared_mem_bytes
    cfg.stream = stream
    return cfg


class Module:
    """cuda.Module (src/cuda.zig:293-316)."""

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def load_embedded(cls) -> "Module":
        h = ctypes.c_void_p()
        check(lib().nc_module_load_embedded(ctypes.byref(h)), "Module.loadData")
        return cls(int(h.value))

    @classmethod
    def load_file(cls, path: str) -> "Module":
        h = ctypes.c_void_p()
        check(lib().nc_module_load_file(ctypes.byref(h), path.encode()), "Module.loadFile")
        return cls(int(h.value))

    def get_function(self, name: str) -> Function:
        f = ctypes.c_void_p()
        check(lib().nc_module_get_function(ctypes.byref(f), self.handle, name.encode()), "Module.getFunction")
        return Function(int(f.value), name)

    def unload(self) -> None:
        if self.handle:
            check(lib().nc_module_unload(self.handle), "Module.unload")
            self.handle = 0


class Stream:
    def __init__(self):
        h = ctypes.c_void_p()
        check(lib().nc_stream_create(ctypes.byref(h)), "Stream.create")
        self.handle = int(h.value)

    def synchronize(self) -> None:
        check(lib().nc_stream_synchronize(self.handle), "Stream.synchronize")

    def destroy(self) -> None:
        if self.handle:
            check(lib().nc_stream_destroy(self.handle), "Stream.destroy")
            self.handle = 0


class Event:
    def __init__(self, timing_only: bool = False):
        """timing_only: nc_event_create_timing (no system-scope cache flush when recorded)."""
        h = ctypes.c_void_p()
        if timing_only:
            check(lib().nc_event_create_timing(ctypes.byref(h)), "Event.createTiming")
        else:
            check(lib().nc_event_create(ctypes.byref(h)), "Event.create")
        self.handle = int(h.value)

    def record(self, stream: Optional[int] = None) -> None:
        check(lib().nc_event_record(self.handle, stream), "Event.record")

    def record_node(self, stream: Optional[int] = None) -> None:
        """nc_event_record_node: under a stream capture, a record node of the captured graph."""
        check(lib().nc_event_record_node(self.handle, stream), "Event.recordNode")

    def synchronize(self) -> None:
        check(lib().nc_event_synchronize(self.handle), "Event.synchronize")

    @staticmethod
    def elapsed(start: "Event", stop: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().nc_event_elapsed(ctypes.byref(ms), start.handle, stop.handle), "Event.elapsed")
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            check(lib().nc_event_destroy(self.handle), "Event.destroy")
            self.handle = 0


class Graph:
    """A captured, instantiated HIP graph (extension; the reference has none)."""

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def capture(cls, stream: "Stream", body) -> "Graph":
        """Capture every launch `body()` issues on `stream` into one replayable graph."""
        check(lib().nc_stream_begin_capture(stream.handle), "Stream.beginCapture")
        try:
            body()
        finally:
            h = ctypes.c_void_p()
            st = lib().nc_stream_end_capture(stream.handle, ctypes.byref(h))
        check(st, "Stream.endCapture")
        return cls(int(h.value))

    def launch(self, stream: "Stream") -> None:
        check(lib().nc_graph_launch(self.handle, stream.handle), "Graph.launch")

    def destroy(self) -> None:
        if self.handle:
            check(lib().nc_graph_destroy(self.handle), "Graph.destroy")
            self.handle = 0


def flash_launch(module: Module, q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, o: DeviceBuffer,
                 opts: FlashOptions, stream: Optional[int] = None, *, q_len: Optional[int] = None,
                 k_len: Optional[int] = None, v_len: Optional[int] = None, o_len: Optional[int] = None,
                 q_offset: int = 0, k_offset: int = 0, v_offset: int = 0, o_offset: int = 0) -> None:
    """flash.launch (src/flash.zig:31-70). Lengths are in elements and default to the buffer size;
    offsets (in elements) let a caller pass a sub-slice, e.g. a deliberately misaligned base.

    Raises ValueError, before anything is launched, when an offset is negative or past the end of
    its buffer, or a length is negative or longer than the elements left after the offset: the C
    ABI's short-buffer check (requireLen) can only trust lengths that describe real memory, and a
    negative one would wrap to ~2^64 in size_t."""
    def span(name, buf, esize, offset, length):
        avail = buf.nbytes // esize
        if offset < 0 or offset > avail:
            raise ValueError(f"flash_launch: {name}_offset {offset} outside the {avail}-element buffer")
        n = avail - offset if length is None else length
        if n < 0 or n > avail - offset:
            raise ValueError(f"flash_launch: {name}_len {n} does not fit the {avail - offset} elements "
                             f"after offset {offset}")
        return n

    ql = span("q", q, 2, q_offset, q_len)
    kl = span("k", k, 2, k_offset, k_len)
    vl = span("v", v, 2, v_offset, v_len)
    ol = span("o", o, 4, o_offset, o_len)
    check(lib().nc_flash_launch_async(module.handle, q.ptr + 2 * q_offset, ql, k.ptr + 2 * k_offset, kl,
                                      v.ptr + 2 * v_offset, vl, o.ptr + 4 * o_offset, ol, ctypes.byref(opts),
                                      stream), "flash.launch")


# ---------------------------------------------------------------------------------------------
# benchmark + host fills
# ---------------------------------------------------------------------------------------------

def benchmark_finish(iter_ms: Sequence[float], bytes_: int = 0, flops: int = 0) -> BenchmarkResult:
    arr = (ctypes.c_float * len(iter_ms))(*iter_ms)
    r = BenchmarkResult()
    lib().nc_benchmark_finish(arr, len(iter_ms), bytes_, flops, ctypes.byref(r))
    return r


def run_kernel(fn: Function, grid, block, params, *, warmup: int = 3, iters: int = 10, bytes_: int = 0,
               flops: int = 0, stream: Optional[int] = None) -> BenchmarkResult:
    """benchmark.runKernel (src/benchmark.zig:35-92)."""
    bo = BenchmarkOptions()
    lib().nc_benchmark_options_init(ctypes.byref(bo))
    bo.warmup_iters = warmup
    bo.iters = iters
    bo.bytes_processed = bytes_
    bo.flops_processed = flops
    bo.stream = stream
    cfg = make_config(grid, block, stream)
    arr = (ctypes.c_void_p * len(params))(*[ctypes.cast(ctypes.pointer(p), ctypes.c_void_p) for p in params])
    r = BenchmarkResult()
    check(lib().nc_benchmark_run_kernel(ctypes.byref(bo), fn.handle, ctypes.byref(cfg), arr, ctypes.byref(r)),
          "benchmark.runKernel")
    return r


def fill_flash_input(n: int, mul: int, add: int, scale: float) -> np.ndarray:
    """fillFlashInput (src/main.zig:1207-1211) as f16 bit patterns."""
    out = np.empty(n, dtype=np.uint16)
    lib().nc_fill_flash_input(out.ctypes.data, n, mul, add, scale)
    return out


def fill_uniform(n: int, seed: int, tensor_id: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().nc_fill_uniform_f16(out.ctypes.data, n, seed, tensor_id, lo, hi)
    return out


def fill_normal(n: int, seed: int, tensor_id: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().nc_fill_normal_f16(out.ctypes.data, n, seed, tensor_id, mean, sigma)
    return out


def fill_uniform_bf16(n: int, seed: int, tensor_id: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    """The draws of fill_uniform rounded to bf16 bit patterns."""
    out = np.empty(n, dtype=np.uint16)
    lib().nc_fill_uniform_bf16(out.ctypes.data, n, seed, tensor_id, lo, hi)
    return out


def fill_normal_bf16(n: int, seed: int, tensor_id: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    """The draws of fill_normal rounded to bf16 bit patterns."""
    out = np.empty(n, dtype=np.uint16)
    lib().nc_fill_normal_bf16(out.ctypes.data, n, seed, tensor_id, mean, sigma)
    return out


def f32_to_bf16(x: float) -> int:
    return int(lib().nc_f32_to_bf16(x))


def bf16_to_f32(h: int) -> float:
    return float(lib().nc_bf16_to_f32(h))


def f32_to_f16(x: float) -> int:
    return int(lib().nc_f32_to_f16(x))


def f16_to_f32(h: int) -> float:
    return float(lib().nc_f16_to_f32(h))


# ---------------------------------------------------------------------------------------------
# Materialized-attention baseline (include/notcute_baselines.h, libnotcute_baselines.so):
# the cublas_materialized case of tools/cuda_baselines.cu:689-759 with rocBLAS GEMMs.
# ---------------------------------------------------------------------------------------------

BASELINES_PATH = os.path.join(HERE, "libnotcute_baselines.so")
MATERIALIZED_MAX_SEQ = 32768
_BASE_SIGS = {
    "nc_materialized_create": (ctypes.c_int, [ctypes.POINTER(_P), _P]),
    "nc_materialized_destroy": (ctypes.c_int, [_P]),
    "nc_materialized_workspace_bytes": (_U64, [ctypes.POINTER(FlashOptions)]),
    "nc_materialized_attention": (
        ctypes.c_int,
        [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, _U64,
         ctypes.POINTER(FlashOptions)]),
    "nc_materialized_last_error": (ctypes.c_char_p, []),
}
_blib: Optional[ctypes.CDLL] = None


def baselines_library(path: str = BASELINES_PATH) -> ctypes.CDLL:
    """Load libnotcute_baselines.so (after libnotcute_flash.so, which it links); raises if unbuilt."""
    global _blib
    if _blib is not None:
        return _blib
    load_library()
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `make -C not-cute-zig_amd` or __graft_entry__.build() first")
    b = ctypes.CDLL(path)
    for name, (res, args) in _BASE_SIGS.items():
        fn = getattr(b, name)
        fn.restype = res
        fn.argtypes = args
    _blib = b
    return b


def _check_base(status: int, what: str) -> None:
    if status != 0:
        detail = (baselines_library().nc_materialized_last_error() or b"").decode(errors="replace")
        raise NcError(status, what, detail)


class Materialized:
    """QK^T GEMM -> softmax kernel -> PV GEMM on one stream (rocBLAS handle bound to it)."""

    def __init__(self, stream: Optional[int] = None):
        h = ctypes.c_void_p()
        _check_base(baselines_library().nc_materialized_create(ctypes.byref(h), stream), "materialized.create")
        self.handle = int(h.value)

    @staticmethod
    def workspace_bytes(opts: FlashOptions) -> int:
        """BH*S*S f32 scores + BH*S*S f16 probabilities; 0 for invalid options."""
        return int(baselines_library().nc_materialized_workspace_bytes(ctypes.byref(opts)))

    def run(self, q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, o: DeviceBuffer, workspace: DeviceBuffer,
            opts: FlashOptions, q_len: Optional[int] = None, k_len: Optional[int] = None,
            v_len: Optional[int] = None, o_len: Optional[int] = None) -> None:
        _check_base(baselines_library().nc_materialized_attention(
            self.handle, q.ptr, q.nbytes // 2 if q_len is None else q_len, k.ptr, k.nbytes // 2 if k_len is None else k_len,
            v.ptr, v.nbytes // 2 if v_len is None else v_len, o.ptr, o.nbytes // 4 if o_len is None else o_len,
            workspace.ptr, workspace.nbytes, ctypes.byref(opts)), "materialized.attention")

    def destroy(self) -> None:
        if self.handle:
            _check_base(baselines_library().nc_materialized_destroy(self.handle), "materialized.destroy")
            self.handle = 0
