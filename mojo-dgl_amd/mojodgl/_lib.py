"""Loads libmdgl.so (the gfx950 kernels) and moves data to and from the GPU.

Replaces the reference's loader (python/mojodgl/_lib.py): the same code
tables and lazy `lib()`, a ctypes signature table for the C ABI declared in
include/mdgl.h, and the value / id ingest rules of its `f64` / `i64`
(_lib.py:127-180), changed in one way: features keep float32 or float64
instead of becoming float64 (every other dtype still becomes float64, with
the reference's rejections of complex values and of integers float64 cannot
hold).

Data movement. numpy arrays (and CPU tensors) are copied to the GPU for the
call and results come back as numpy arrays (CPU tensors); torch tensors on
the GPU are used in place and results stay on the GPU. torch is used only for
device memory, copies and the current stream; every kernel is libmdgl.so's.
There is no CPU fallback: without a visible GPU a call that would launch a
kernel raises RuntimeError.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import subprocess
import threading

import numpy as np
import torch  # loads the HIP runtime libmdgl.so then binds to

from .base import DGLError

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(ROOT, "csrc")
LIB = os.environ.get("MOJODGL_LIB") or os.path.join(ROOT, "lib", "libmdgl.so")


class BuildError(RuntimeError):
    pass


# codes of src/ported.mojo:44-65 (the same values cross the C ABI)
SRC_CODE, DST_CODE, EDGE_CODE = 0, 1, 2
OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_DOT = 0, 1, 2, 3, 4
OP_COPY_LHS, OP_COPY_RHS = 5, 6
REDUCE_SUM, REDUCE_MAX, REDUCE_MIN, REDUCE_MEAN = 0, 1, 2, 3

BINARY_OPS = {"add": OP_ADD, "sub": OP_SUB, "mul": OP_MUL, "div": OP_DIV, "dot": OP_DOT}
REDUCERS = {"sum": REDUCE_SUM, "max": REDUCE_MAX, "min": REDUCE_MIN, "mean": REDUCE_MEAN}
TARGETS = {"u": SRC_CODE, "v": DST_CODE, "e": EDGE_CODE}

FLOAT32, FLOAT64 = 0, 1
REPLACE_INF = 1
RHS_CSR_ORDER = 2
LHS_LINE_ROWS = 8  # mdgl_gspmm: lhs rows copied to start on 128-byte lines
NARROW_SLABS = 32  # mdgl_gspmm: 32-lane column slabs for wide rows (a local graph)
COO_LOCALITY_BLOCKS = 1024  # counts written by mdgl_coo_locality
SEGMENTS_SHORT = 4  # mdgl_segment_reduce: no segment longer than SEGMENT_SPLIT_ROWS
SEGMENTS_SKIP_LONG = 8  # mdgl_segment_reduce: longer segments left for a LONG_ONLY call
SEGMENTS_LONG_ONLY = 16  # mdgl_segment_reduce: only the segments longer than SEGMENT_SPLIT_ROWS
SEGMENT_SPLIT_ROWS = 4096
EINVAL, EWORKSPACE, ENOTSUP = -1, -2, -3  # negative statuses of include/mdgl.h

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_C = ctypes.c_int

# name -> (argtypes, restype), as declared in include/mdgl.h
_SIGNATURES = {
    "mdgl_last_error": ([], ctypes.c_char_p),
    "mdgl_workers": ([], _I64),
    "mdgl_trace_ranges": ([], _C),
    "mdgl_cumsum": ([_P, _P, _I64, _P], _C),
    "mdgl_segment_offsets": ([_P, _I64, _I64, _P, _P, _P, _I64, _P], _C),
    "mdgl_segment_offsets_workspace_bytes": ([_I64], _I64),
    "mdgl_replace_inf_with_zero": ([_P, _P, _I64, _C, _P], _C),
    "mdgl_clamp_i64": ([_P, _P, _I64, _I64, _I64, _P], _C),
    "mdgl_gsddmm": ([_P, _P, _P, _P, _P, _I64, _C, _C, _C, _I64, _I64, _I64, _C, _P, _P, _C, _P],
                    _C),
    "mdgl_gspmm": ([_P, _P, _P, _P, _P, _P, _I64, _C, _I64, _I64, _I64, _C, _P, _C, _P, _P, _P,
                    _P, _P, _P, _I64, _I32, _P, _P, _I64, _P, _I64, _C, _C, _P], _C),
    "mdgl_gspmm_rows": ([_P, _P, _P, _P, _P, _P, _I64, _C, _I64, _I64, _I64, _C, _P, _C, _P,
                         _P, _P, _P, _P, _I64, _C, _C, _P], _C),
    "mdgl_gspmm_workspace_bytes": ([_I64, _I64, _C, _C], _I64),
    "mdgl_gspmm_lanes": ([_C, _I64, _I64, _I64, _C, _P, _P, _P, _P, _C, _C, _P, _P], _C),
    "mdgl_coo_locality": ([_P, _P, _I64, _I64, _P, _P], _C),
    "mdgl_edge_softmax_positional": ([_P, _I64, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P, _P, _P,
                                      _P, _I64, _C, _P], _C),
    "mdgl_edge_softmax_positional_workspace_bytes": ([_I64, _I64, _I64, _P, _P, _C], _I64),
    "mdgl_read_stream": ([_P, _I64, _P, _P], _C),
    "mdgl_read_stream_sink_bytes": ([_I64], _I64),
    "mdgl_read_rows": ([_P, _I64, _I64, _P, _I64, _P, _I64, _P, _P], _C),
    "mdgl_read_rows_sink_bytes": ([_I64], _I64),
    "mdgl_gspmm_noalloc": ([_P, _P, _P, _P, _P, _P, _I64, _C, _I64, _I64, _I64, _C, _P, _C, _P, _P,
                            _P, _P, _P, _P, _I64, _I32, _P, _P, _I64, _C, _C, _P], _C),
    "mdgl_gspmm_mul_sum_dot": ([_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _C, _P,
                                _P, _P, _P, _I64, _I32, _P, _P, _I64, _P, _I64, _C, _P], _C),
    "mdgl_segment_reduce": ([_P, _P, _P, _I64, _I64, _C, _I64, _C, _C, _P], _C),
    "mdgl_segment_reduce_arg": ([_P, _P, _P, _P, _I64, _I64, _C, _I64, _C, _C, _P], _C),
    "mdgl_segment_ids": ([_P, _I64, _I64, _P, _P], _C),
    "mdgl_softmax_geometry": ([_I64, _C, _P, _P, _P, _P], _C),
    "mdgl_softmax_workspace_bytes": ([_I64, _I64, _I64, _C], _I64),
    "mdgl_segment_softmax": ([_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _C, _P, _P, _P, _P,
                              _I64, _I64, _P, _I64, _C, _P], _C),
    "mdgl_segment_softmax_short": ([_P, _P, _P, _I64, _I64, _I64, _C, _P], _C),
    "mdgl_edge_softmax_": ([_P, _P, _P, _P, _P, _P, _P, _I64, _C, _I64, _P, _P, _C, _P, _P, _P,
                            _P, _I64, _I64, _P, _I64, _P, _I64, _C, _P], _C),
    "mdgl_segment_mm": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _C, _P], _C),
    "mdgl_segment_mm_workspace_bytes": ([_I64, _I64, _I64, _I64, _C], _I64),
    "mdgl_gather_mm": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _C, _P], _C),
    "mdgl_gather_mm_workspace_bytes": ([_I64, _I64, _I64, _I64, _C], _I64),
    "mdgl_segment_mm_grad": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _C, _P],
                             _C),
    "mdgl_segment_mm_grad_workspace_bytes": ([_I64, _I64, _I64, _I64, _C], _I64),
    "mdgl_gather_mm_grad": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _C, _P],
                            _C),
    "mdgl_gather_mm_grad_workspace_bytes": ([_I64, _I64, _I64, _I64, _C], _I64),
    "mdgl_build_csr": ([_P, _P, _I64, _I64, _P, _P, _P, _P, _I64, _P], _C),
    "mdgl_build_csr_workspace_bytes": ([_I64, _I64], _I64),
    "mdgl_gspmm_edge_grad": ([_P, _P, _P, _P, _P, _I64, _I64, _C, ctypes.c_double, _C, _P], _C),
    "mdgl_rows_by_degree": ([_P, _P, _P, _I64, _I64, _C, _P], _C),
    "mdgl_scale": ([_P, _P, _I64, ctypes.c_double, _C, _P], _C),
    "mdgl_keep_where": ([_P, _P, _P, _I64, _C, _P], _C),
    "mdgl_gather_rows": ([_P, _P, _P, _I64, _I64, _C, _P], _C),
    "mdgl_scatter_rows": ([_P, _P, _P, _I64, _I64, _C, _P], _C),
    "mdgl_edge_softmax_grad": ([_P, _P, _P, _P, _P, _I64, _I64, _C, _P], _C),
}


def _sources_digest() -> str:
    """sha256 of what libmdgl.so is built from, in the Makefile's order
    (`STAMPED`: the csrc sources sorted by name, the C ABI header, the
    Makefile); the build writes the same digest to LIB + '.sources'."""
    names = sorted(n for n in os.listdir(CSRC) if n.endswith((".hip", ".h", ".cpp")))
    paths = [os.path.join(CSRC, n) for n in names]
    paths += [os.path.join(os.path.dirname(ROOT), "include", "mdgl.h"),
              os.path.join(CSRC, "Makefile")]
    h = hashlib.sha256()
    for path in paths:
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def is_current(path: str = None) -> bool:
    """Whether the library at `path` (default LIB) exists and was built from
    the sources as they are now."""
    path = path or LIB
    try:
        with open(path + ".sources") as f:
            stamp = f.read().strip()
    except OSError:
        return False
    return os.path.exists(path) and stamp == _sources_digest()


def build(force: bool = False) -> str:
    """Compile csrc/ into LIB with hipcc when it is missing or stale (its
    source stamp differs from the sources), or always with `force`; as the
    reference's build (_lib.py:89-110). MOJODGL_LIB names another output
    path. Raises BuildError when the compiler fails."""
    if not force and is_current():
        return LIB
    cmd = ["make", "-C", CSRC, "-j8", "OUT=" + os.path.abspath(LIB)]
    if force:
        cmd.insert(1, "-B")
    try:
        proc = subprocess.run(cmd, capture_output=True, text=True, timeout=1800)
        if proc.returncode == 0 and not force and not is_current():
            # make found every target newer than its prerequisites while the
            # digest differs (a source deleted or renamed, or one restored
            # with an older time): rebuild everything once
            proc = subprocess.run(cmd[:1] + ["-B"] + cmd[1:], capture_output=True, text=True,
                                  timeout=1800)
    except OSError as exc:  # no make
        raise BuildError("cannot run make: {}".format(exc)) from exc
    if proc.returncode != 0 or not is_current():
        raise BuildError("building {} failed:\n{}".format(
            LIB, (proc.stderr or proc.stdout).strip()[-4000:]))
    return LIB


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded libmdgl.so, built first if it is missing or stale (the
    reference's lazy build, _lib.py:116-124)."""
    global _lib
    if _lib is None:
        handle = ctypes.CDLL(build())
        for name, (argtypes, restype) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Raise for a non-zero status of a libmdgl call."""
    if rc == 0:
        return
    msg = lib().mdgl_last_error().decode(errors="replace")
    if rc < 0:
        raise DGLError("{}: {}".format(what, msg))
    raise RuntimeError("{} failed on the GPU: {}".format(what, msg))


# ------------------------------------------------------------------ device
_GPU_SEEN = False
_CUDA = torch.device("cuda")  # the current device, resolved at each use


def device() -> torch.device:
    """The current GPU (loud error when there is none; checked until one is seen)."""
    global _GPU_SEEN
    if not _GPU_SEEN:
        if not torch.cuda.is_available():
            raise RuntimeError(
                "mojodgl runs its kernels on an AMD GPU through libmdgl.so and no GPU is visible")
        _GPU_SEEN = True
    return _CUDA


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)


def current_device() -> int:
    """Index of the current GPU (torch's; cheap once torch's GPU state is up)."""
    if _get_device is not None and _GPU_SEEN:
        return _get_device()
    return torch.cuda.current_device()


def stream() -> int:
    """torch's current stream on the current device, as a raw hipStream_t."""
    if _raw_stream is not None:
        return _raw_stream(current_device())
    return torch.cuda.current_stream().cuda_stream


_PINNED = threading.local()


def _side_stream(dev: int) -> torch.cuda.Stream:
    """A second stream per thread and device (default priority) for small
    copies that should not sit between the caller's kernels."""
    streams = getattr(_PINNED, "side", None)
    if streams is None:
        streams = _PINNED.side = {}
    st = streams.get(dev)
    if st is None:
        st = streams[dev] = torch.cuda.Stream(device=dev)
    return st


class Readback:
    """A small GPU int64 tensor copied to pinned host memory without waiting:
    the GPU goes on with what the caller queues next, and values() waits for
    the copy only. With `after` (an event recorded on the current stream right
    after the kernel that writes `src`), the copy runs on a side stream behind
    that event, so kernels the caller queued since then do not wait for it;
    otherwise it follows the work queued so far on the current stream. One
    pinned buffer per thread, device and purpose, reused across calls."""

    def __init__(self, src: torch.Tensor, purpose: str, after=None):
        bufs = getattr(_PINNED, "bufs", None)
        if bufs is None:
            bufs = _PINNED.bufs = {}
        dev = src.device.index if src.device.index is not None else current_device()
        key = (purpose, dev, src.numel())
        buf = bufs.get(key)
        if buf is None:
            buf = bufs[key] = torch.empty(src.numel(), dtype=torch.int64, pin_memory=True)
        self._buf, self._src = buf, src  # src lives until the copy is done
        self._done = torch.cuda.Event()
        if after is None:
            buf.copy_(src.reshape(-1), non_blocking=True)
            self._done.record()
        else:
            side = _side_stream(dev)
            side.wait_event(after)
            with torch.cuda.stream(side):
                buf.copy_(src.reshape(-1), non_blocking=True)
                self._done.record(side)
            src.record_stream(side)  # its memory is not reused before the copy is done

    def values(self) -> list:
        self._done.synchronize()
        self._src = None
        return self._buf.tolist()


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------ values
_F32, _F64 = np.dtype(np.float32), np.dtype(np.float64)
_TORCH_TO_NP = {torch.float32: _F32, torch.float64: _F64}
_NP_TO_TORCH = {_F32: torch.float32, _F64: torch.float64}


class Feat:
    """A validated feature operand: a float32/float64 numpy array or tensor."""

    __slots__ = ("data", "is_torch", "device", "shape", "dtype")

    def __init__(self, data, is_torch, dev):
        self.data = data
        self.is_torch = is_torch
        self.device = dev
        self.shape = tuple(data.shape)
        self.dtype = _TORCH_TO_NP[data.dtype] if is_torch else data.dtype

    @property
    def ndim(self):
        return len(self.data.shape)


def _check_int_exact(a: np.ndarray) -> None:
    # every integer dtype but int64 must survive float64 exactly (_lib.py:144-161)
    if np.issubdtype(a.dtype, np.integer) and a.dtype != np.int64 and a.size:
        with np.errstate(invalid="ignore"):
            back = a.astype(np.float64).astype(a.dtype)
        if not bool(np.array_equal(back, a)):
            raise DGLError("{} values do not survive the conversion to float64 exactly".format(
                a.dtype))


def feature(a) -> Feat:
    """Validate a feature operand without touching the GPU."""
    if isinstance(a, Feat):
        return a
    if isinstance(a, torch.Tensor):
        if a.is_complex():
            raise DGLError("complex features are not supported")
        if a.dtype in (torch.float32, torch.float64):
            t = a
        elif a.dtype in (torch.float16, torch.bfloat16):
            t = a.to(torch.float32)
        else:
            if a.dtype != torch.bool and a.dtype != torch.int64:
                _check_int_exact(a.detach().cpu().numpy())
            t = a.to(torch.float64)
        return Feat(t, True, a.device)
    arr = np.asanyarray(a)
    if np.iscomplexobj(arr):
        raise DGLError("complex features are not supported")
    if arr.dtype == np.float32 or arr.dtype == np.float64:
        out = np.ascontiguousarray(arr)
    elif arr.dtype == np.float16:
        out = np.ascontiguousarray(arr, dtype=np.float32)
    else:
        _check_int_exact(arr)
        out = np.ascontiguousarray(arr, dtype=np.float64)
    return Feat(out, False, None)


def common_dtype(*feats) -> np.dtype:
    """float32 when every given operand is float32, else float64."""
    seen = False
    for f in feats:
        if f is not None:
            if f.dtype != _F32:
                return _F64
            seen = True
    return _F32 if seen else _F64


def dtype_code(dtype) -> int:
    if dtype is _F32:
        return FLOAT32
    return FLOAT32 if np.dtype(dtype) == _F32 else FLOAT64


def torch_dtype(dtype) -> torch.dtype:
    t = _NP_TO_TORCH.get(dtype) if isinstance(dtype, np.dtype) else None
    if t is not None:
        return t
    return torch.float32 if np.dtype(dtype) == _F32 else torch.float64


def on_device(f: Feat, dtype) -> torch.Tensor:
    """The operand as a contiguous GPU tensor of `dtype` (copied if needed)."""
    dev = device()
    tdt = torch_dtype(dtype)
    if f.is_torch:
        t = f.data
        if t.is_cuda and t.dtype == tdt and t.is_contiguous() \
                and t.get_device() == current_device():
            return t
    else:
        t = torch.from_numpy(f.data)
    return t.to(device=dev, dtype=tdt).contiguous()


def wants_torch(*feats) -> bool:
    return any(f is not None and f.is_torch for f in feats)


def out_device(*feats):
    for f in feats:
        if f is not None and f.is_torch:
            return f.device
    return None


def give_back(t: torch.Tensor, as_torch: bool, dev):
    """A result tensor in the caller's container: numpy, or a tensor on `dev`."""
    if as_torch:
        return t if dev is None or t.device == dev else t.to(dev)
    return t.cpu().numpy()


# ------------------------------------------------------------------ ids
def i64(a) -> np.ndarray:
    """Node ids / lengths as C-contiguous int64 numpy (reference _lib.py:166-180)."""
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    a = np.asanyarray(a)
    if np.issubdtype(a.dtype, np.floating) and a.size:
        if not bool(np.all(a == np.floor(a))):
            raise DGLError("node ids and segment lengths must be whole numbers, got {}".format(
                a.dtype))
    return np.ascontiguousarray(a, dtype=np.int64)


def i64_device(a) -> torch.Tensor:
    """Ids / lengths as a contiguous int64 GPU tensor. A GPU tensor is
    converted where it lies (no host round trip); anything else goes through
    `i64` and is uploaded."""
    if isinstance(a, torch.Tensor) and a.device.type == "cuda":
        if a.is_complex():
            raise DGLError("node ids and segment lengths must be whole numbers, got {}".format(
                a.dtype))
        if a.is_floating_point() and a.numel() and bool((a != torch.floor(a)).any()):
            raise DGLError("node ids and segment lengths must be whole numbers, got {}".format(
                a.dtype))
        return a.detach().to(device=device(), dtype=torch.int64).contiguous()
    return torch.from_numpy(i64(a)).to(device())


def settle() -> None:
    """Wait until the work queued so far on the current stream has run. A
    graph's lazily built device structures (endpoints, CSR schedules,
    softmax plans) are cached only after this, so a call on another stream
    or thread that finds them cached reads them complete. Once per
    structure; these builds therefore belong before a HIP graph capture (the
    CSR build reads its row pointers back anyway)."""
    torch.cuda.current_stream().synchronize()


def i32_device(a: np.ndarray) -> torch.Tensor:
    """An int64 host index array as an int32 GPU tensor (values checked < 2**31)."""
    if a.size and (int(a.max()) >= 2 ** 31 or int(a.min()) < -2 ** 31):
        raise DGLError("index values must fit in int32 on the GPU")
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(device())


def main() -> int:
    print(build(force=False))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
