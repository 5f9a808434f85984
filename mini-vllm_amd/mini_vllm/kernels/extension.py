"""Build and load the MI355X kernel library, and bind it as the reference's extension.

The reference JIT-compiles ``csrc/*.cu`` into a pybind11 module ``mini_vllm_C`` with
``torch.utils.cpp_extension`` for sm_120 (mini_vllm/kernels/extension.py:266-298) and
calls it with torch tensors. Here the kernels are HIP for gfx950 behind a plain C ABI
(``include/minivllm_hip.h``), built with ``hipcc`` into ``libminivllm_hip.so`` and bound
with :mod:`ctypes`. :func:`load_extension` returns an object exposing the reference
module's functions -- ``paged_attention``, ``rmsnorm``, ``rope``, ``swiglu``, ``hello``
-- with the same arguments and refusal messages, so ``ops.py`` and every caller above
it are unchanged.

Ownership follows the reference: each call returns a freshly allocated output tensor
(torch's caching allocator), so the library itself never allocates device memory. The
split-K workspace of ``paged_attention`` is a torch allocation kept here, one per
(device, stream), grown on demand. Work goes on torch's current stream and nothing
synchronizes.
"""

from __future__ import annotations

import ctypes
import hashlib
import math
import os
import subprocess
import sys
import threading
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path
from typing import Any

import torch

PACKAGE_ROOT = Path(__file__).resolve().parents[2]  # .../mini-vllm_amd
CSRC_DIR = PACKAGE_ROOT / "csrc"
BUILD_DIR = PACKAGE_ROOT / "_build"
LIB_DIR = PACKAGE_ROOT / "lib"
# MVLLM_LIBRARY points the loader at another build of the same library (variant builds
# for measurements); the default is the in-tree build.
LIB_PATH = Path(os.environ.get("MVLLM_LIBRARY") or LIB_DIR / "libminivllm_hip.so")
REPO_ROOT = PACKAGE_ROOT.parent
INCLUDE_DIR = REPO_ROOT / "include"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed fp32 VALU ops are disabled for every kernel: the compiler emits them from
# ordinary float code otherwise.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]

# Per-source extra flags. The elementwise kernels must round exactly where the
# reference's PyTorch expressions round, so FMA contraction is off there; the decode
# kernels form the step's new token with the same QK-norm + RoPE code, which then has
# to compile to the same bits (measured: contraction left on there moved one in ten
# float16 rows by an ulp, and the decode ran no faster).
EXTRA_FLAGS = {"elementwise.hip": ["-ffp-contract=off"], "linear.hip": ["-ffp-contract=off"],
               "paged_decode.hip": ["-ffp-contract=off"]}

# hipBLASLt (csrc/blas.hip). Its soname is the one torch's bundled copy carries, so in a
# process that has imported torch the library binds to that copy.
LINK_LIBS = ["-L/opt/rocm/lib", "-lhipblaslt"]

ABI_VERSION = 15

DTYPE_CODES: dict[torch.dtype, int] = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.float8_e4m3fn: 3,
}

_lock = threading.Lock()
_extension: "HipExtension | None" = None


class ToolchainError(RuntimeError):
    """Raised when the library cannot be built or loaded."""


# ----------------------------------------------------------------------- build


def sources() -> list[Path]:
    found = sorted(CSRC_DIR.glob("*.hip"))
    if not found:
        raise ToolchainError(f"no HIP sources found in {CSRC_DIR}")
    return found


def source_hash() -> str | None:
    """16 hex digits of a SHA-256 over the kernel sources, their headers and the build
    flags: the identity the build stamps into the library (``mvllm_build_id``). None
    when the sources are not beside the package (an installed library)."""
    files = sorted(CSRC_DIR.glob("*.hip")) + sorted(CSRC_DIR.glob("*.hpp")) + sorted(
        INCLUDE_DIR.glob("*.h"))
    if not any(f.suffix == ".hip" for f in files):
        return None
    h = hashlib.sha256()
    h.update(repr((HIP_FLAGS, sorted(EXTRA_FLAGS.items()), LINK_LIBS)).encode())
    for f in files:
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()[:16]


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link ``lib/libminivllm_hip.so``.

    Always compiles (this is the "does it build" check); objects go to ``_build/``
    and the library is replaced atomically so a running process never maps a
    half-written file.
    """
    if not Path(HIPCC).exists():
        raise ToolchainError(f"hipcc not found at {HIPCC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    stamp = f'-DMVLLM_SOURCE_HASH="{source_hash()}"'

    def compile_one(src: Path) -> Path:
        obj = BUILD_DIR / (src.stem + ".o")
        extra = [*EXTRA_FLAGS.get(src.name, []), *([stamp] if src.name == "capi.hip" else [])]
        cmd = [HIPCC, *HIP_FLAGS, *extra, f"-I{INCLUDE_DIR}", "-c",
               str(src), "-o", str(obj)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        noise = "'-packed-fp32-ops' is not a recognized feature"
        log = "\n".join(l for l in (result.stderr + result.stdout).splitlines() if noise not in l)
        if result.returncode != 0:
            raise ToolchainError(f"hipcc failed on {src.name}:\n{log}")
        if verbose and log.strip():
            print(log, file=sys.stderr)
        return obj

    workers = jobs or min(8, os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(compile_one, sources()))

    tmp = LIB_PATH.with_suffix(f".so.tmp{os.getpid()}")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), *LINK_LIBS,
           "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise ToolchainError(f"link failed:\n{result.stderr}{result.stdout}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


# ------------------------------------------------------------------- bindings


class _DenseArgs(ctypes.Structure):
    """``mvllm_dense_args`` of include/minivllm_hip.h."""

    _fields_ = [
        ("out", ctypes.c_void_p),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_stride_batch", ctypes.c_int64),
        ("k_stride_head", ctypes.c_int64),
        ("k_stride_pos", ctypes.c_int64),
        ("v_stride_batch", ctypes.c_int64),
        ("v_stride_head", ctypes.c_int64),
        ("v_stride_pos", ctypes.c_int64),
        ("batch", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("query_len", ctypes.c_int32),
        ("kv_len", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class _PlanOptions(ctypes.Structure):
    """``mvllm_plan_options`` of include/minivllm_hip.h (0 = the planner's choice)."""

    _fields_ = [
        ("decode_schedule", ctypes.c_int32),
        ("decode_wgs_per_cu", ctypes.c_int32),
        ("decode_waves_per_cu", ctypes.c_int32),
        ("decode_split_tokens", ctypes.c_int32),
        ("prefill_schedule", ctypes.c_int32),
        ("prefill_wgs_per_cu", ctypes.c_int32),
        ("prefill_staging", ctypes.c_int32),
        ("prefill_share_tiles", ctypes.c_int32),
        ("prefill_pieces", ctypes.c_int32),
        ("prefill_piece_pct", ctypes.c_int32),
    ]


SCHEDULES = {"stream": 1, "grid": 2}


def make_plan_options(options: dict[str, Any] | None) -> "_PlanOptions | None":
    """``mvllm_plan_options`` from a dict of its field names (schedules may be given as
    "stream" / "grid"); None for the planner's defaults."""
    if not options:
        return None
    fields = {name for name, _ in _PlanOptions._fields_}
    unknown = set(options) - fields
    if unknown:
        raise ValueError(f"unknown plan options {sorted(unknown)}; known: {sorted(fields)}")
    values = {k: SCHEDULES.get(v, v) if k.endswith("schedule") else int(v)
              for k, v in options.items()}
    return _PlanOptions(**values)


class _Plan(ctypes.Structure):
    _fields_ = [
        ("decode_mode", ctypes.c_int32),
        ("decode_workgroups", ctypes.c_int32),
        ("split_tokens", ctypes.c_int32),
        ("prefill_mfma", ctypes.c_int32),
        ("workspace_bytes", ctypes.c_uint64),
        ("prefill_workgroups", ctypes.c_int32),
        ("prefill_pieces", ctypes.c_int32),
    ]


class _BlasChoice(ctypes.Structure):
    """``mvllm_blas_choice`` of include/minivllm_hip.h."""

    _fields_ = [
        ("candidates", ctypes.c_int32),
        ("timed", ctypes.c_int32),
        ("chosen", ctypes.c_int32),
        ("first_us", ctypes.c_float),
        ("chosen_us", ctypes.c_float),
    ]


DECODE_MODES = {0: "none", 1: "stream", 2: "grid", 3: "by_row"}


def _bind(lib: ctypes.CDLL) -> None:
    p, i32, i64, u64, f32 = (
        ctypes.c_void_p,
        ctypes.c_int32,
        ctypes.c_int64,
        ctypes.c_uint64,
        ctypes.c_float,
    )
    lib.mvllm_last_error.restype = ctypes.c_char_p
    lib.mvllm_last_error.argtypes = []
    lib.mvllm_abi_version.restype = ctypes.c_int
    lib.mvllm_abi_version.argtypes = []
    lib.mvllm_build_id.restype = ctypes.c_char_p
    lib.mvllm_build_id.argtypes = []
    opts = ctypes.POINTER(_PlanOptions)
    lib.mvllm_paged_attention_plan.restype = ctypes.c_int
    lib.mvllm_paged_attention_plan.argtypes = [i32] * 10 + [opts, ctypes.POINTER(_Plan)]
    lib.mvllm_dense_attention_plan.restype = ctypes.c_int
    lib.mvllm_dense_attention_plan.argtypes = [ctypes.POINTER(_DenseArgs), ctypes.POINTER(ctypes.c_uint64)]
    lib.mvllm_dense_attention.restype = ctypes.c_int
    lib.mvllm_dense_attention.argtypes = [ctypes.POINTER(_DenseArgs), p, ctypes.c_uint64, p]
    lib.mvllm_paged_attention.restype = ctypes.c_int
    lib.mvllm_paged_attention.argtypes = (
        [p] * 10 + [i32] * 6 + [i64, i32, i32, i32, f32, i32, i32, opts, p, u64, p]
    )
    lib.mvllm_paged_attention_noalloc.restype = ctypes.c_int
    lib.mvllm_paged_attention_noalloc.argtypes = (
        [p] * 10 + [i32] * 6 + [i64, i32, i32, i32, f32, i32, i32, opts, p]
    )
    lib.mvllm_rmsnorm.restype = ctypes.c_int
    lib.mvllm_rmsnorm.argtypes = [p, p, p, i64, i64, f32, i32, p]
    lib.mvllm_embed_rmsnorm.restype = ctypes.c_int
    lib.mvllm_embed_rmsnorm.argtypes = [p, p, p, i64, p, p, p, i64, i32, p, f32, i32, p]
    lib.mvllm_add_rmsnorm.restype = ctypes.c_int
    lib.mvllm_add_rmsnorm.argtypes = [p, p, p, p, p, i64, i32, f32, i32, p]
    lib.mvllm_rope.restype = ctypes.c_int
    lib.mvllm_rope.argtypes = [p, p, p, i32, p, p, i64, i64, i64, i64, i64, i32, p]
    lib.mvllm_swiglu.restype = ctypes.c_int
    lib.mvllm_swiglu.argtypes = [p, p, p, i64, i32, p]
    lib.mvllm_swiglu_interleaved.restype = ctypes.c_int
    lib.mvllm_swiglu_interleaved.argtypes = [p, p, i64, i64, i32, p]
    lib.mvllm_axpby.restype = ctypes.c_int
    lib.mvllm_axpby.argtypes = [p, p, f32, f32, i64, p]
    lib.mvllm_qk_norm_rope.restype = ctypes.c_int
    lib.mvllm_qk_norm_rope.argtypes = [p] * 7 + [i32, p, p, i64, i32, i32, i32, i64, i64, f32, i32, p]
    lib.mvllm_qk_norm_rope_kv_write.restype = ctypes.c_int
    lib.mvllm_qk_norm_rope_kv_write.argtypes = (
        [p] * 9 + [i32, p, p, p, i64, i64, i32, i32, i32, i64, i64, f32, i64, i64, i32, p])
    lib.mvllm_paged_decode_qk_norm_rope.restype = ctypes.c_int
    lib.mvllm_paged_decode_qk_norm_rope.argtypes = (
        [p] * 4 + [i64, i64] + [p] * 4 + [i64, f32] + [p] * 6 + [i32] * 5
        + [i64, i32, i32, f32, i32, opts, p, u64, p])
    lib.mvllm_kv_write.restype = ctypes.c_int
    lib.mvllm_kv_write.argtypes = [p] * 7 + [i32] * 4 + [i64, i32, i32, p]
    lib.mvllm_argmax.restype = ctypes.c_int
    lib.mvllm_argmax.argtypes = [p, p, i64, i64, i64, i32, p, u64, p]
    lib.mvllm_argmax_workspace_bytes.restype = u64
    lib.mvllm_argmax_workspace_bytes.argtypes = [i64, i64]
    lib.mvllm_linear_pack.restype = ctypes.c_int
    lib.mvllm_linear_pack.argtypes = [p, p, i64, i64, i32, p]
    lib.mvllm_linear_workspace_bytes.restype = u64
    lib.mvllm_linear_workspace_bytes.argtypes = [i64, i64, i64]
    lib.mvllm_linear.restype = ctypes.c_int
    lib.mvllm_linear.argtypes = [p, p, p, i64, i64, i64, i32, p, u64, p]
    lib.mvllm_linear_split.restype = ctypes.c_int
    lib.mvllm_linear_split.argtypes = [p, p, p, p, p, i64, i64, i64, i64, i64, i32, p, u64, p]
    lib.mvllm_linear_residual.restype = ctypes.c_int
    lib.mvllm_linear_residual.argtypes = [p, p, p, p, i64, i64, i64, i32, p, u64, p]
    lib.mvllm_linear_swiglu.restype = ctypes.c_int
    lib.mvllm_linear_swiglu.argtypes = [p, p, p, i64, i64, i64, i32, p, u64, p]
    lib.mvllm_linear_residual_rmsnorm.restype = ctypes.c_int
    lib.mvllm_linear_residual_rmsnorm.argtypes = [p, p, p, p, p, p, i64, i64, i64, f32, i32, p, u64, p]
    lib.mvllm_blas_linear.restype = ctypes.c_int
    lib.mvllm_blas_linear.argtypes = [p, p, p, i64, i64, i64, i32, p, u64, p]
    lib.mvllm_blas_workspace_bytes.restype = u64
    lib.mvllm_blas_workspace_bytes.argtypes = []
    lib.mvllm_blas_plans_cached.restype = ctypes.c_int
    lib.mvllm_blas_plans_cached.argtypes = []
    lib.mvllm_read_probe.restype = ctypes.c_int
    lib.mvllm_read_probe.argtypes = [p, i64, p, i64, i64, i32, p, i64, p]
    lib.mvllm_split_stats.restype = None
    lib.mvllm_split_stats.argtypes = [ctypes.POINTER(i32), ctypes.POINTER(i64), ctypes.POINTER(i64)]
    lib.mvllm_blas_tune.restype = ctypes.c_int
    lib.mvllm_blas_tune.argtypes = [p, p, p, i64, i64, i64, i32, p, u64, p, ctypes.POINTER(i32)]
    lib.mvllm_blas_tuning.restype = ctypes.c_int
    lib.mvllm_blas_tuning.argtypes = [i64, i64, i64, i32, ctypes.POINTER(_BlasChoice)]



EXPORTED_SYMBOLS = (
    "mvllm_last_error",
    "mvllm_abi_version",
    "mvllm_build_id",
    "mvllm_paged_attention_plan",
    "mvllm_paged_attention",
    "mvllm_paged_attention_noalloc",
    "mvllm_rmsnorm",
    "mvllm_rope",
    "mvllm_swiglu",
    "mvllm_swiglu_interleaved",
    "mvllm_add_rmsnorm",
    "mvllm_embed_rmsnorm",
    "mvllm_axpby",
    "mvllm_kv_write",
    "mvllm_qk_norm_rope",
    "mvllm_argmax",
    "mvllm_qk_norm_rope_kv_write",
    "mvllm_paged_decode_qk_norm_rope",
    "mvllm_argmax_workspace_bytes",
    "mvllm_dense_attention_plan",
    "mvllm_dense_attention",
    "mvllm_linear_pack",
    "mvllm_linear_workspace_bytes",
    "mvllm_linear_residual_rmsnorm",
    "mvllm_linear",
    "mvllm_linear_split",
    "mvllm_linear_residual",
    "mvllm_linear_swiglu",
    "mvllm_blas_linear",
    "mvllm_blas_workspace_bytes",
    "mvllm_blas_plans_cached",
    "mvllm_blas_tuning",
    "mvllm_blas_tune",
    "mvllm_split_stats",
    "mvllm_read_probe",
)


def open_library(path: Path = LIB_PATH) -> ctypes.CDLL:
    """dlopen the library and declare its signatures (no GPU needed).

    The in-tree library must have been built from the sources beside it: its stamped
    build id is compared with :func:`source_hash` and a stale build is refused (a
    library named by ``MVLLM_LIBRARY`` is the caller's choice and only warned about).
    """
    if not path.exists():
        raise ToolchainError(
            f"{path} is not built; run `python -m mini_vllm.kernels.extension --build` "
            "or __graft_entry__.build()"
        )
    lib = ctypes.CDLL(str(path))
    _bind(lib)
    version = lib.mvllm_abi_version()
    if version != ABI_VERSION:
        raise ToolchainError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    built, current = lib.mvllm_build_id().decode(), source_hash()
    if current is not None and built != current:
        message = (f"{path} was built from other sources (build id {built}, sources "
                   f"{current}); rebuild it: __graft_entry__.build()")
        if path == LIB_DIR / "libminivllm_hip.so":
            raise ToolchainError(message)
        print(f"warning: {message}", file=sys.stderr)
    return lib


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    """The raw HIP stream torch's current stream of ``device`` wraps. Read through
    torch's raw accessor: building a Stream object per op costs ~4 us of host time,
    which an eager prefill iteration pays for every one of its ~400 launches."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


class HipExtension:
    """The reference's ``mini_vllm_C`` module surface, served by libminivllm_hip.so."""

    def __init__(self, lib: ctypes.CDLL) -> None:
        self.lib = lib
        self.path = LIB_PATH
        self._workspaces: dict[tuple[int, int], torch.Tensor] = {}
        self._recording: list[torch.Tensor] | None = None

    def workspace(self, device: torch.device, nbytes: int) -> torch.Tensor:
        """The kernels' workspace of (device, current stream), grown on demand (paged and
        dense attention, split projections).

        Kept rather than allocated per call so a steady decode loop (or a captured
        graph) reuses one buffer; calls on one stream are ordered, so they never race.
        A buffer outgrown is dropped (torch's allocator frees it in stream order); a
        captured graph keeps the buffers its launches name alive itself, through
        :meth:`recording_workspaces`.
        """
        key = (device.index if device.index is not None else torch.cuda.current_device(),
               _stream(device))
        ws = self._workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            size = max(nbytes, 2 * ws.numel() if ws is not None else 0)
            size = (size + (1 << 20) - 1) >> 20 << 20
            ws = torch.empty(size, dtype=torch.uint8, device=device)
            self._workspaces[key] = ws
        if self._recording is not None:
            self._recording.append(ws)
        return ws

    def recording_workspaces(self):
        """Context manager yielding the list of every workspace handed out inside it:
        a graph capture holds that list for as long as the graph lives, since its
        launches name those buffers."""
        ext = self

        class _Recorder:
            def __enter__(self):
                self.previous, ext._recording = ext._recording, []
                return ext._recording

            def __exit__(self, *exc):
                ext._recording = self.previous
                return False

        return _Recorder()

    # -- plumbing
    def _check(self, rc: int) -> None:
        if rc != 0:
            message = self.lib.mvllm_last_error().decode(errors="replace")
            raise RuntimeError(message or f"libminivllm_hip call failed with code {rc}")

    # -- ops
    def hello(self, x: torch.Tensor, a: float, b: float) -> torch.Tensor:
        """``a * x + b`` (reference csrc/hello.cu), the toolchain smoke test."""
        if not x.is_cuda:
            raise RuntimeError("hello: x must be a CUDA tensor")
        if x.dtype != torch.float32:
            raise RuntimeError("hello: x must be float32")
        x = x.contiguous()
        out = torch.empty_like(x)
        self._check(self.lib.mvllm_axpby(out.data_ptr(), x.data_ptr(), a, b, x.numel(), _stream(x.device)))
        return out

    @staticmethod
    def add_rmsnorm_supported(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor) -> bool:
        """Whether ``add_rmsnorm`` serves these tensors (the library's own rule: f32, f16
        or bf16 alike, CUDA, rows of whole 16-byte chunks, at most 512 of them)."""
        e = 4 if x.dtype == torch.float32 else 8
        dim = x.shape[-1] if x.dim() else 0
        return (x.dtype in (torch.float32, torch.float16, torch.bfloat16) and x.is_cuda
                and residual.dtype == x.dtype and weight.dtype == x.dtype
                and residual.shape == x.shape and weight.shape == (dim,)
                and dim > 0 and dim % e == 0 and dim // e <= 512)

    def add_rmsnorm(self, x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                    eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
        """``h = residual + x`` (torch's rounding) and ``rmsnorm(h)`` in one launch;
        returns (h, normed)."""
        if not (residual.is_cuda and weight.is_cuda) or not self.add_rmsnorm_supported(x, residual, weight):
            raise RuntimeError("add_rmsnorm: x, residual and weight must be CUDA tensors of one "
                               "dtype (f32, f16, bf16), x and residual alike, rows of whole "
                               "16-byte chunks (at most 512)")
        x, residual, weight = x.contiguous(), residual.contiguous(), weight.contiguous()
        h = torch.empty_like(x)
        out = torch.empty_like(x)
        dim = x.shape[-1]
        self._check(self.lib.mvllm_add_rmsnorm(h.data_ptr(), out.data_ptr(), x.data_ptr(),
                                               residual.data_ptr(), weight.data_ptr(),
                                               x.numel() // dim, dim, float(eps),
                                               DTYPE_CODES[x.dtype], _stream(x.device)))
        return h, out

    @staticmethod
    def embed_rmsnorm_supported(table: torch.Tensor, ids: torch.Tensor, weight: torch.Tensor,
                                index: torch.Tensor | None = None,
                                prev: torch.Tensor | None = None) -> bool:
        """Whether ``embed_rmsnorm`` serves these tensors: a contiguous 2-D table of f32,
        f16 or bf16 on the GPU with rows of whole 16-byte chunks (at most 512), the
        weight alike, 1-D int64 ids (and index of the same length, with prev) on the
        same device."""
        e = 4 if table.dtype == torch.float32 else 8
        dim = table.shape[-1] if table.dim() == 2 else 0

        def i64(t):
            return t.dtype == torch.int64 and t.dim() == 1 and t.device == table.device
        return (table.dtype in (torch.float32, torch.float16, torch.bfloat16) and table.is_cuda
                and table.is_contiguous() and weight.dtype == table.dtype
                and weight.shape == (dim,) and dim > 0 and dim % e == 0 and dim // e <= 512
                and i64(ids) and (index is None or (prev is not None and i64(index) and i64(prev)
                                                    and index.shape == ids.shape)))

    def embed_rmsnorm(self, table: torch.Tensor, ids: torch.Tensor, weight: torch.Tensor,
                      eps: float = 1e-6, index: torch.Tensor | None = None,
                      prev: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """``h`` = the table rows of the tokens (row i: ``prev[index[i]]`` where ``index``
        is given and ``index[i] >= 0``, else ``ids[i]``) and ``rmsnorm(h)`` in one launch;
        returns (h, normed). A token id outside the table gives NaN rows."""
        if not self.embed_rmsnorm_supported(table, ids, weight, index, prev):
            raise RuntimeError("embed_rmsnorm: a contiguous f32/f16/bf16 CUDA table with rows "
                               "of whole 16-byte chunks (at most 512), its weight, and 1-D "
                               "int64 ids (and an index of their length, with prev) on its "
                               "device")
        ids = ids.contiguous()
        if index is not None:
            index, prev = index.contiguous(), prev.contiguous()
        rows = ids.shape[0]
        h = torch.empty(rows, table.shape[1], dtype=table.dtype, device=table.device)
        out = torch.empty_like(h)
        self._check(self.lib.mvllm_embed_rmsnorm(
            h.data_ptr(), out.data_ptr(), table.data_ptr(), table.shape[0], ids.data_ptr(),
            _ptr(index), _ptr(prev), rows, table.shape[1], weight.contiguous().data_ptr(),
            float(eps), DTYPE_CODES[table.dtype], _stream(table.device)))
        return h, out

    def rmsnorm(self, x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
        """RMSNorm over the last dim (reference csrc/rmsnorm.cu:121-169)."""
        if not x.is_cuda:
            raise RuntimeError("rmsnorm: x must be a CUDA tensor")
        if not weight.is_cuda:
            raise RuntimeError("rmsnorm: weight must be a CUDA tensor")
        if x.dim() < 1:
            raise RuntimeError("rmsnorm: x must have at least one dimension")
        if weight.dim() != 1:
            raise RuntimeError(f"rmsnorm: weight must be 1-D, got {weight.dim()} dimensions")
        if x.shape[-1] != weight.shape[0]:
            raise RuntimeError(
                f"rmsnorm: x's last dimension is {x.shape[-1]} but weight has "
                f"{weight.shape[0]} elements"
            )
        if x.dtype == torch.float64:
            raise RuntimeError(
                "rmsnorm: float64 is not supported; this kernel accumulates in fp32, which "
                "would silently lose precision. Use the PyTorch path."
            )
        if x.dtype != weight.dtype:
            raise RuntimeError(
                f"rmsnorm: x is {x.dtype} but weight is {weight.dtype}; the PyTorch path "
                "promotes mixed dtypes, this kernel does not"
            )
        code = DTYPE_CODES.get(x.dtype)
        if code is None or code == 3:
            raise RuntimeError(f"rmsnorm: dtype {x.dtype} is not supported")
        x = x.contiguous()
        weight = weight.contiguous()
        out = torch.empty_like(x)
        dim = x.shape[-1]
        rows = 0 if dim == 0 else x.numel() // dim
        self._check(
            self.lib.mvllm_rmsnorm(
                out.data_ptr(), x.data_ptr(), weight.data_ptr(), rows, dim, eps, code, _stream(x.device)
            )
        )
        return out

    def rope(
        self, x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
    ) -> torch.Tensor:
        """Rotate-halves RoPE at explicit positions (reference csrc/rope.cu:115-195)."""
        if not x.is_cuda:
            raise RuntimeError("rope: x must be a CUDA tensor")
        if not positions.is_cuda:
            raise RuntimeError("rope: positions must be a CUDA tensor")
        if not (cos.is_cuda and sin.is_cuda):
            raise RuntimeError("rope: the cos/sin tables must be CUDA tensors")
        if x.dtype == torch.float64:
            raise RuntimeError(
                "rope: float64 is not supported; this kernel computes the rotation in fp32. "
                "Use the PyTorch path."
            )
        if x.dim() < 3:
            raise RuntimeError(
                "rope: x must be N.. x H x D — a head axis is required, since one position "
                f"applies to every head of a token. Got {x.dim()} dimensions"
            )
        dim = x.shape[-1]
        if dim % 2 != 0:
            raise RuntimeError(f"rope: the head dimension must be even, got {dim}")
        if cos.dim() != 2 or sin.dim() != 2:
            raise RuntimeError("rope: the cos/sin tables must be 2-D")
        if cos.shape != sin.shape:
            raise RuntimeError(f"rope: cos is {tuple(cos.shape)} but sin is {tuple(sin.shape)}")
        if cos.shape[1] != dim:
            raise RuntimeError(
                f"rope: the tables are {cos.shape[1]} wide but the head dimension is {dim}; "
                "they are built as max_seq_len x D with the angles duplicated"
            )
        if cos.dtype != torch.float32 or sin.dtype != torch.float32:
            raise RuntimeError(
                "rope: the cos/sin tables must be float32 even when x is bf16. "
                f"Got {cos.dtype}"
            )
        if positions.dtype not in (torch.int32, torch.int64):
            raise RuntimeError(f"rope: positions must be int32 or int64, got {positions.dtype}")
        code = DTYPE_CODES.get(x.dtype)
        if code is None or code == 3:
            raise RuntimeError(f"rope: dtype {x.dtype} is not supported")
        x = x.contiguous()
        out = torch.empty_like(x)
        rows = 0 if dim == 0 else x.numel() // dim
        if rows == 0:
            return out
        positions = positions.contiguous()
        cos = cos.contiguous()
        sin = sin.contiguous()
        heads = x.shape[-2]
        tokens = rows // heads
        count = positions.numel()
        if count == 0:
            raise RuntimeError("rope: positions is empty")
        if tokens % count != 0:
            raise RuntimeError(
                f"rope: x holds {tokens} tokens, which is not a multiple of the {count} "
                "positions given, so the positions cannot broadcast over it"
            )
        self._check(
            self.lib.mvllm_rope(
                out.data_ptr(),
                x.data_ptr(),
                positions.data_ptr(),
                positions.element_size(),
                cos.data_ptr(),
                sin.data_ptr(),
                rows,
                heads,
                dim,
                count,
                cos.shape[0],
                code,
                _stream(x.device),
            )
        )
        return out

    def kv_write(self, key_pool: torch.Tensor, value_pool: torch.Tensor, key: torch.Tensor,
                 value: torch.Tensor, slot_mapping: torch.Tensor, *,
                 k_scale: torch.Tensor | None = None,
                 v_scale: torch.Tensor | None = None) -> None:
        """Scatter ``T x H_k x D`` keys/values into one layer's pools at ``slot_mapping``
        (replaces the reference's ``index_copy_`` pair, block/kv_pool.py:116-155). An
        fp8 pool is quantised per (block, kv head) and its ``k_scale``/``v_scale``
        (``num_blocks x H_k`` fp32) are updated in place; see include/minivllm_hip.h."""
        tensors = (key_pool, value_pool, key, value, slot_mapping)
        if not all(t.is_cuda for t in tensors):
            raise RuntimeError("kv_write: pools, keys, values and slot_mapping must be CUDA tensors")
        if key_pool.dim() != 4 or key_pool.shape != value_pool.shape:
            raise RuntimeError("kv_write: the pools must be num_blocks x P x H_k x D and match")
        nb, bs, hk, d = key_pool.shape
        if key.shape != value.shape or key.dim() != 3 or tuple(key.shape[1:]) != (hk, d):
            raise RuntimeError(
                f"kv_write: expected keys and values shaped T x {hk} x {d}, got "
                f"{tuple(key.shape)} and {tuple(value.shape)}")
        if slot_mapping.dtype != torch.int32 or slot_mapping.shape != (key.shape[0],):
            raise RuntimeError("kv_write: slot_mapping must be int32 with one slot per token")
        if not (key_pool.is_contiguous() and value_pool.is_contiguous()):
            raise RuntimeError("kv_write: the pools must be contiguous")
        if key.dtype != value.dtype:
            raise RuntimeError(f"kv_write: keys are {key.dtype} but values are {value.dtype}")
        fp8 = key_pool.dtype == torch.float8_e4m3fn
        if fp8:
            for name, sc in (("k_scale", k_scale), ("v_scale", v_scale)):
                if sc is None or sc.dtype != torch.float32 or tuple(sc.shape) != (nb, hk) \
                        or not sc.is_contiguous() or not sc.is_cuda:
                    raise RuntimeError(
                        f"kv_write: a float8 pool needs {name} as a contiguous float32 "
                        f"{nb} x {hk} CUDA tensor")
        elif k_scale is not None or v_scale is not None:
            raise RuntimeError("kv_write: k_scale / v_scale are for float8 pools only")
        key = key.contiguous()
        value = value.contiguous()
        slot_mapping = slot_mapping.contiguous()
        src = DTYPE_CODES.get(key.dtype, -1)
        pool = DTYPE_CODES.get(key_pool.dtype, -1)
        self._check(self.lib.mvllm_kv_write(
            key_pool.data_ptr(), value_pool.data_ptr(),
            k_scale.data_ptr() if fp8 else None, v_scale.data_ptr() if fp8 else None,
            key.data_ptr(), value.data_ptr(), slot_mapping.data_ptr(),
            key.shape[0], hk, d, bs, nb, src, pool, _stream(key.device)))

    @staticmethod
    def linear_packable(w: torch.Tensor) -> bool:
        """Whether ``linear_pack`` takes ``w``: a contiguous f16/bf16 N x K device matrix,
        K a multiple of 64 up to 65536, 16-byte aligned."""
        return (w.dim() == 2 and w.is_cuda and w.dtype in (torch.float16, torch.bfloat16)
                and w.shape[1] % 64 == 0 and 64 <= w.shape[1] <= 65536 and w.is_contiguous()
                and w.data_ptr() % 16 == 0)

    def linear_pack(self, w: torch.Tensor) -> torch.Tensor:
        """``w`` (N x K) pre-shuffled into the skinny kernels' fragment order: a flat
        tensor of ceil(N / 32) * 32 * K elements (``torch_path.pack_fragments``)."""
        if not self.linear_packable(w):
            raise RuntimeError(f"linear_pack: w {tuple(w.shape)} {w.dtype} is not packable (a "
                               "contiguous f16/bf16 device matrix, K a multiple of 64 up to 65536)")
        n, k = w.shape
        packed = torch.empty(-(-n // 32) * 32 * k, dtype=w.dtype, device=w.device)
        self._check(self.lib.mvllm_linear_pack(packed.data_ptr(), w.data_ptr(), n, k,
                                               DTYPE_CODES[w.dtype], _stream(w.device)))
        return packed

    def linear_supported(self, x: torch.Tensor, w_packed: torch.Tensor, n: int) -> bool:
        """Whether the skinny projection kernel serves ``x`` @ W.T for W (n x K) packed as
        ``w_packed``: at most 64 contiguous rows of f16/bf16, K a multiple of 64 up to
        65536, 16-byte-aligned operands."""
        if x.dim() != 2 or x.dtype != w_packed.dtype or not (x.is_cuda and w_packed.is_cuda):
            return False
        if x.dtype not in (torch.float16, torch.bfloat16):
            return False
        m, k = x.shape
        return (1 <= m <= 64 and k % 64 == 0 and k <= 65536 and n >= 1
                and w_packed.numel() == -(-n // 32) * 32 * k and x.is_contiguous()
                and w_packed.is_contiguous() and x.data_ptr() % 16 == 0
                and w_packed.data_ptr() % 16 == 0)

    def _require(self, name: str, x: torch.Tensor, w_packed: torch.Tensor, n: int) -> None:
        if not self.linear_supported(x, w_packed, n):
            raise RuntimeError(
                f"{name}: x {tuple(x.shape)} {x.dtype} with a packed {n}-row weight of "
                f"{w_packed.numel()} {w_packed.dtype} elements is not served by the skinny kernel "
                "(at most 64 contiguous f16/bf16 rows, K a multiple of 64 up to 65536)")

    def _linear_ws(self, x: torch.Tensor, n: int) -> tuple[int, int]:
        """(pointer, bytes) of the partial-sum workspace of x (M x K) against n rows of
        weights: none for K <= 1024, else the stream's shared workspace."""
        need = int(self.lib.mvllm_linear_workspace_bytes(x.shape[0], n, x.shape[1]))
        if need == 0:
            return 0, 0
        ws = self.workspace(x.device, need)
        return ws.data_ptr(), ws.numel()

    def linear(self, x: torch.Tensor, w_packed: torch.Tensor, n: int) -> torch.Tensor:
        """``x @ W.T`` for ``x`` M x K (M <= 64) and W (n x K) packed: the skinny projection
        kernel (fp32 accumulation, one rounding)."""
        self._require("linear", x, w_packed, n)
        y = torch.empty((x.shape[0], n), dtype=x.dtype, device=x.device)
        self._check(self.lib.mvllm_linear(y.data_ptr(), x.data_ptr(), w_packed.data_ptr(),
                                          x.shape[0], n, x.shape[1], DTYPE_CODES[x.dtype],
                                          *self._linear_ws(x, n), _stream(x.device)))
        return y

    def linear_split(self, x: torch.Tensor, w_packed: torch.Tensor,
                     sizes: tuple[int, ...]) -> tuple[torch.Tensor, ...]:
        """``x @ W.T`` with its columns cut into contiguous outputs of ``sizes`` (up to
        three; all but the last multiples of 32): the q, k, v projections in one launch."""
        if not 1 <= len(sizes) <= 3 or any(s % 32 for s in sizes[:-1]) or min(sizes) < 0:
            raise RuntimeError(f"linear_split: column groups {sizes}: one to three, all but the "
                               "last multiples of 32")
        self._require("linear_split", x, w_packed, sum(sizes))
        outs = [torch.empty((x.shape[0], n), dtype=x.dtype, device=x.device) for n in sizes]
        ptrs = [o.data_ptr() for o in outs] + [0] * (3 - len(outs))
        ns = list(sizes) + [0] * (3 - len(sizes))
        self._check(self.lib.mvllm_linear_split(*ptrs, x.data_ptr(), w_packed.data_ptr(),
                                                x.shape[0], *ns, x.shape[1], DTYPE_CODES[x.dtype],
                                                *self._linear_ws(x, sum(sizes)), _stream(x.device)))
        return tuple(outs)

    def linear_residual(self, x: torch.Tensor, w_packed: torch.Tensor,
                        residual: torch.Tensor) -> torch.Tensor:
        """``residual + x @ W.T`` in one launch (W has ``residual.shape[1]`` rows), each
        step rounded as torch rounds it."""
        n = residual.shape[-1]
        self._require("linear_residual", x, w_packed, n)
        if residual.shape != (x.shape[0], n) or residual.dtype != x.dtype or not residual.is_contiguous():
            raise RuntimeError(f"linear_residual: residual must be a contiguous {x.shape[0]} x {n} "
                               f"{x.dtype} tensor, got {tuple(residual.shape)} {residual.dtype}")
        y = torch.empty_like(residual)
        self._check(self.lib.mvllm_linear_residual(y.data_ptr(), x.data_ptr(), w_packed.data_ptr(),
                                                   residual.data_ptr(), x.shape[0], n, x.shape[1],
                                                   DTYPE_CODES[x.dtype], *self._linear_ws(x, n),
                                                   _stream(x.device)))
        return y

    def linear_swiglu(self, x: torch.Tensor, w_packed: torch.Tensor, n_out: int) -> torch.Tensor:
        """``swiglu(x @ gate.T, x @ up.T)`` in one launch, over
        ``torch_path.interleave_gate_up(gate, up)`` (2 n_out rows) packed."""
        if n_out % 16:
            raise RuntimeError(f"linear_swiglu: {n_out} output columns, not a multiple of 16")
        self._require("linear_swiglu", x, w_packed, 2 * n_out)
        y = torch.empty((x.shape[0], n_out), dtype=x.dtype, device=x.device)
        self._check(self.lib.mvllm_linear_swiglu(y.data_ptr(), x.data_ptr(), w_packed.data_ptr(),
                                                 x.shape[0], n_out, x.shape[1], DTYPE_CODES[x.dtype],
                                                 *self._linear_ws(x, 2 * n_out), _stream(x.device)))
        return y

    @staticmethod
    def linear_residual_rmsnorm_supported(x: torch.Tensor, n: int) -> bool:
        """Whether ``linear_residual_rmsnorm`` serves x (M x K) against n weight rows:
        K > 1024 and n a multiple of 512 up to 4096 (beyond ``linear_supported``)."""
        return x.dim() == 2 and x.shape[1] > 1024 and n % 512 == 0 and n <= 4096

    def linear_residual_rmsnorm(self, x: torch.Tensor, w_packed: torch.Tensor,
                                residual: torch.Tensor, norm_weight: torch.Tensor,
                                eps: float) -> tuple[torch.Tensor, torch.Tensor]:
        """(h, normed): h = residual + x @ W.T and normed = rmsnorm(h, norm_weight, eps),
        each bit for bit its unfused op, in two launches."""
        n = residual.shape[-1]
        self._require("linear_residual_rmsnorm", x, w_packed, n)
        if not self.linear_residual_rmsnorm_supported(x, n):
            raise RuntimeError(f"linear_residual_rmsnorm: N={n} K={x.shape[1]} is not served "
                               "(K > 1024, N a multiple of 512 up to 4096)")
        if (residual.shape != (x.shape[0], n) or residual.dtype != x.dtype or not residual.is_contiguous()
                or norm_weight.shape != (n,) or norm_weight.dtype != x.dtype
                or not norm_weight.is_contiguous()):
            raise RuntimeError("linear_residual_rmsnorm: residual must be a contiguous M x N tensor "
                               "and norm_weight a contiguous N vector, both of x's dtype")
        h = torch.empty_like(residual)
        normed = torch.empty_like(residual)
        self._check(self.lib.mvllm_linear_residual_rmsnorm(
            h.data_ptr(), normed.data_ptr(), x.data_ptr(), w_packed.data_ptr(), residual.data_ptr(),
            norm_weight.data_ptr(), x.shape[0], n, x.shape[1], float(eps), DTYPE_CODES[x.dtype],
            *self._linear_ws(x, n), _stream(x.device)))
        return h, normed

    @staticmethod
    def blas_linear_supported(x: torch.Tensor, w: torch.Tensor) -> bool:
        """Whether :meth:`blas_linear` serves ``x @ w.T``: device tensors, 2-D, contiguous,
        16-byte aligned, fp16 / bf16 of one dtype, K >= 1."""
        return (x.dim() == 2 and w.dim() == 2 and x.dtype == w.dtype
                and x.dtype in (torch.float16, torch.bfloat16) and x.shape[1] == w.shape[1]
                and x.shape[1] >= 1 and x.is_cuda and w.device == x.device
                and x.is_contiguous() and w.is_contiguous()
                and (x.data_ptr() | w.data_ptr()) % 16 == 0)

    def blas_linear(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor | None:
        """``x @ w.T`` through the library's hipBLASLt entry (descriptors and algorithm
        kept per shape), or None when hipBLASLt has no algorithm for the shape (the
        caller takes torch's product). Unserved operands raise."""
        if not self.blas_linear_supported(x, w):
            raise RuntimeError(f"blas_linear: x {tuple(x.shape)} {x.dtype} and w {tuple(w.shape)} "
                               f"{w.dtype} are not served (2-D contiguous 16-byte aligned device "
                               "fp16 or bf16 of one dtype, matching K)")
        y = torch.empty((x.shape[0], w.shape[0]), dtype=x.dtype, device=x.device)
        ws = self.workspace(x.device, int(self.lib.mvllm_blas_workspace_bytes()))
        rc = self.lib.mvllm_blas_linear(y.data_ptr(), x.data_ptr(), w.data_ptr(), x.shape[0],
                                        w.shape[0], x.shape[1], DTYPE_CODES[x.dtype],
                                        ws.data_ptr(), ws.numel(), _stream(x.device))
        if rc == 2:  # MVLLM_ERR_UNSUPPORTED: no algorithm for this shape
            return None
        self._check(rc)
        return y

    def blas_plans_cached(self) -> int:
        """Shapes the hipBLASLt entry currently keeps."""
        return int(self.lib.mvllm_blas_plans_cached())

    def read_probe(self, base: torch.Tensor, page_bytes: int, page_ids: torch.Tensor | None,
                   workgroups: int, sink: torch.Tensor) -> None:
        """Read pages of ``base`` (a device buffer) with the library's read-only probe:
        ``page_ids`` (device int32, each < base bytes / page_bytes) or every page in
        address order; ``sink`` (device uint8/int32) receives one word per lane. For
        the benchmark's bandwidth ceiling; enqueued on the current stream."""
        nbytes = base.numel() * base.element_size()
        num_pages = page_ids.numel() if page_ids is not None else nbytes // page_bytes
        if page_ids is not None and (page_ids.dtype != torch.int32 or not page_ids.is_contiguous()):
            raise RuntimeError("read_probe: page_ids must be contiguous int32")
        self._check(self.lib.mvllm_read_probe(
            base.data_ptr(), nbytes, _ptr(page_ids), num_pages, page_bytes, workgroups,
            sink.data_ptr(), sink.numel() * sink.element_size() // 4, _stream(base.device)))

    def split_stats(self) -> dict[str, int]:
        """The split prefill grid's counter regions in use on the current device, and the
        split launches that ran every item whole (no region left; stream capturing)."""
        used, no_region, capturing = ctypes.c_int32(0), ctypes.c_int64(0), ctypes.c_int64(0)
        self.lib.mvllm_split_stats(ctypes.byref(used), ctypes.byref(no_region),
                                   ctypes.byref(capturing))
        return {"regions_used": used.value, "whole_no_region": no_region.value,
                "whole_capturing": capturing.value}

    def blas_tune(self, x: torch.Tensor, w: torch.Tensor) -> int:
        """Time every hipBLASLt algorithm for ``x @ w.T`` at x's row count and keep the
        fastest as extra candidates for every later choice of w's shape
        (``mvllm_blas_tune``; ~0.5 s, waits on the host, not under graph capture).
        Returns the algorithms timed."""
        if not self.blas_linear_supported(x, w):
            raise RuntimeError(f"blas_tune: x {tuple(x.shape)} {x.dtype} and w {tuple(w.shape)} "
                               f"{w.dtype} are not served")
        y = torch.empty((x.shape[0], w.shape[0]), dtype=x.dtype, device=x.device)
        ws = self.workspace(x.device, int(self.lib.mvllm_blas_workspace_bytes()))
        timed = ctypes.c_int32(0)
        self._check(self.lib.mvllm_blas_tune(y.data_ptr(), x.data_ptr(), w.data_ptr(), x.shape[0],
                                             w.shape[0], x.shape[1], DTYPE_CODES[x.dtype],
                                             ws.data_ptr(), ws.numel(), _stream(x.device),
                                             ctypes.byref(timed)))
        return int(timed.value)

    def blas_choice(self, m: int, n: int, k: int, dtype: torch.dtype) -> dict[str, Any]:
        """How the hipBLASLt entry chose the algorithm it keeps for (m, n, k, dtype) on the
        current device: the heuristic's candidates, how many were timed, the kept one's
        index in the heuristic's order, and the first's and the kept one's us per product
        (-1 untimed)."""
        out = _BlasChoice()
        self._check(self.lib.mvllm_blas_tuning(m, n, k, DTYPE_CODES[dtype], ctypes.byref(out)))
        return {f: getattr(out, f) for f, _ in _BlasChoice._fields_}

    def qk_norm_rope_supported(self, dtype: torch.dtype, head_dim: int) -> bool:
        """Whether the fused kernel serves this dtype / head dim (16-byte chunks per head
        a power of two from 2 to 64)."""
        n = {torch.float32: 4, torch.float16: 8, torch.bfloat16: 8}.get(dtype)
        if n is None or head_dim % n:
            return False
        return head_dim // n in (2, 4, 8, 16, 32, 64)

    @staticmethod
    def _qk_norm_rope_checks(name: str, q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                             k_weight: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                             sin: torch.Tensor) -> int:
        """The shape, dtype and device rules both fused QK-norm + RoPE entries share
        (the kernel takes q's token count for k, v and the slots, and reads the tables
        at pos x D); returns q's dtype code."""
        tensors = (q, k, q_weight, k_weight, positions, cos, sin)
        if not all(t.is_cuda for t in tensors):
            raise RuntimeError(f"{name}: every tensor must be a CUDA tensor")
        if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
            raise RuntimeError(
                f"{name}: q must be T x H_q x D and k T x H_k x D, got {tuple(q.shape)} "
                f"and {tuple(k.shape)}")
        d = q.shape[2]
        if q.dtype != k.dtype or q_weight.dtype != q.dtype or k_weight.dtype != q.dtype:
            raise RuntimeError(f"{name}: q, k and both weights must share a dtype")
        if q_weight.shape != (d,) or k_weight.shape != (d,):
            raise RuntimeError(f"{name}: the weights must be [{d}]")
        if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape \
                or cos.dim() != 2 or cos.shape[1] != d:
            raise RuntimeError(f"{name}: the cos/sin tables must be float32 max_pos x {d}")
        if positions.dtype not in (torch.int32, torch.int64) or positions.dim() != 1:
            raise RuntimeError(f"{name}: positions must be a 1-D int32 or int64 tensor")
        code = DTYPE_CODES.get(q.dtype)
        if code is None or code == 3:
            raise RuntimeError(f"{name}: dtype {q.dtype} is not supported")
        return code

    def qk_norm_rope(self, q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                     k_weight: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                     sin: torch.Tensor, eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
        """Per-head RMSNorm then RoPE of q ``T x H_q x D`` and k ``T x H_k x D`` in one
        launch, bitwise equal to ``rope(rmsnorm(x, w))`` with this library's kernels."""
        code = self._qk_norm_rope_checks("qk_norm_rope", q, k, q_weight, k_weight, positions,
                                         cos, sin)
        d = q.shape[2]
        q, k = q.contiguous(), k.contiguous()
        q_out, k_out = torch.empty_like(q), torch.empty_like(k)
        if q.shape[0] == 0:
            return q_out, k_out
        positions = positions.contiguous()
        self._check(self.lib.mvllm_qk_norm_rope(
            q_out.data_ptr(), k_out.data_ptr(), q.data_ptr(), k.data_ptr(),
            q_weight.contiguous().data_ptr(), k_weight.contiguous().data_ptr(),
            positions.data_ptr(), positions.element_size(), cos.contiguous().data_ptr(),
            sin.contiguous().data_ptr(), q.shape[0], q.shape[1], k.shape[1], d,
            positions.numel(), cos.shape[0], float(eps), code, _stream(q.device)))
        return q_out, k_out

    def qk_norm_rope_kv_write(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              q_weight: torch.Tensor, k_weight: torch.Tensor,
                              positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                              eps: float, key_pool: torch.Tensor, value_pool: torch.Tensor,
                              slot_mapping: torch.Tensor) -> torch.Tensor:
        """``qk_norm_rope`` whose rotated k, and v, go straight to their slots of the
        layer's paged pools (``num_blocks x P x H_k x D`` of q's dtype) in the same
        launch; returns the rotated q. q, k and v may be column views of one fused
        projection's output: heads contiguous within a token, any 16-byte-aligned token
        stride (k and v sharing theirs)."""
        name = "qk_norm_rope_kv_write"
        code = self._qk_norm_rope_checks(name, q, k, q_weight, k_weight, positions, cos, sin)
        if not (key_pool.is_cuda and value_pool.is_cuda and v.is_cuda and slot_mapping.is_cuda):
            raise RuntimeError("qk_norm_rope_kv_write: every tensor must be a CUDA tensor")
        if (key_pool.dtype != q.dtype or value_pool.dtype != q.dtype or v.dtype != q.dtype
                or key_pool.shape != value_pool.shape or key_pool.dim() != 4
                or tuple(key_pool.shape[2:]) != tuple(k.shape[1:]) or v.shape != k.shape
                or not (key_pool.is_contiguous() and value_pool.is_contiguous())):
            raise RuntimeError(
                "qk_norm_rope_kv_write: the pools must be contiguous num_blocks x P x H_k x D "
                f"tensors of q's dtype matching k and v, got {tuple(key_pool.shape)} "
                f"{key_pool.dtype} for k {tuple(k.shape)}")
        if slot_mapping.dtype != torch.int32 or slot_mapping.shape != (k.shape[0],) \
                or not slot_mapping.is_contiguous():
            raise RuntimeError(f"{name}: slot_mapping must be a contiguous int32 [T]")
        d = q.shape[2]

        def rows_ok(t):  # heads contiguous within each token
            return t.stride(2) == 1 and t.stride(1) == d
        if not (rows_ok(q) and rows_ok(k) and rows_ok(v)) or k.stride(0) != v.stride(0):
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        q_out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        if q.shape[0] == 0:
            return q_out
        positions = positions.contiguous()
        self._check(self.lib.mvllm_qk_norm_rope_kv_write(
            q_out.data_ptr(), key_pool.data_ptr(), value_pool.data_ptr(), q.data_ptr(),
            k.data_ptr(), v.data_ptr(), q_weight.contiguous().data_ptr(),
            k_weight.contiguous().data_ptr(), positions.data_ptr(), positions.element_size(),
            cos.contiguous().data_ptr(), sin.contiguous().data_ptr(), slot_mapping.data_ptr(),
            key_pool.shape[0] * key_pool.shape[1],
            q.shape[0], q.shape[1], k.shape[1], d, positions.numel(), cos.shape[0], float(eps),
            q.stride(0), k.stride(0), code, _stream(q.device)))
        return q_out

    def swiglu_interleaved(self, gate_up: torch.Tensor) -> torch.Tensor:
        """``swiglu`` over ``gate_up`` [T, 2 I], the fused gate/up projection's output in
        the 16-column interleave of ``torch_path.interleave_gate_up``; returns [T, I]."""
        if not gate_up.is_cuda or gate_up.dim() != 2 or gate_up.shape[1] % 32 != 0:
            raise RuntimeError("swiglu_interleaved: gate_up must be a CUDA [T, 2 I] tensor, "
                               "I a multiple of 16")
        code = DTYPE_CODES.get(gate_up.dtype)
        if code is None or code == 3:
            raise RuntimeError(f"swiglu_interleaved: dtype {gate_up.dtype} is not supported")
        gate_up = gate_up.contiguous()
        rows, cols = gate_up.shape[0], gate_up.shape[1] // 2
        out = torch.empty(rows, cols, dtype=gate_up.dtype, device=gate_up.device)
        self._check(self.lib.mvllm_swiglu_interleaved(out.data_ptr(), gate_up.data_ptr(), rows,
                                                      cols, code, _stream(gate_up.device)))
        return out

    def swiglu(self, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
        """``silu(gate) * up`` (reference csrc/swiglu.cu:87-120)."""
        if not (gate.is_cuda and up.is_cuda):
            raise RuntimeError("swiglu: gate and up must be CUDA tensors")
        if gate.shape != up.shape:
            raise RuntimeError(
                f"swiglu: gate is {tuple(gate.shape)} but up is {tuple(up.shape)}; they are the "
                "two projections of the same tokens and must match"
            )
        if gate.dtype != up.dtype:
            raise RuntimeError(f"swiglu: gate is {gate.dtype} but up is {up.dtype}")
        if gate.dtype == torch.float64:
            raise RuntimeError(
                "swiglu: float64 is not supported; this kernel evaluates the sigmoid in fp32. "
                "Use the PyTorch path."
            )
        code = DTYPE_CODES.get(gate.dtype)
        if code is None or code == 3:
            raise RuntimeError(f"swiglu: dtype {gate.dtype} is not supported")
        gate = gate.contiguous()
        up = up.contiguous()
        out = torch.empty_like(gate)
        if gate.numel() == 0:
            return out
        self._check(
            self.lib.mvllm_swiglu(
                out.data_ptr(), gate.data_ptr(), up.data_ptr(), gate.numel(), code, _stream(gate.device)
            )
        )
        return out

    def argmax(self, logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """``logits.argmax(dim=-1)`` (int64) for a 2-D f32/f16/bf16 device tensor whose
        rows are contiguous: torch's order (NaN highest, -0 == +0, first index wins).
        ``out``: a contiguous int64 [rows] device tensor to write (default: a new one)."""
        if not logits.is_cuda or logits.dim() != 2 or logits.stride(1) != 1:
            raise RuntimeError("argmax: expected a 2-D CUDA tensor with contiguous rows, got "
                               f"{tuple(logits.shape)} strides {logits.stride()}")
        if logits.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise RuntimeError(f"argmax: dtype {logits.dtype} is not served (f32, f16, bf16)")
        if out is None:
            out = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
        elif (out.dtype != torch.int64 or out.shape != (logits.shape[0],) or not out.is_contiguous()
              or out.device != logits.device):
            raise RuntimeError(f"argmax: out must be a contiguous int64 [{logits.shape[0]}] tensor "
                               "on the logits' device")
        if logits.shape[0] == 0:
            return out
        rows, vocab = logits.shape
        need = int(self.lib.mvllm_argmax_workspace_bytes(rows, vocab))
        ws = self.workspace(logits.device, need) if need else None
        self._check(self.lib.mvllm_argmax(out.data_ptr(), logits.data_ptr(), rows, vocab,
                                          max(logits.stride(0), vocab), DTYPE_CODES[logits.dtype],
                                          ws.data_ptr() if ws is not None else 0, need,
                                          _stream(logits.device)))
        return out

    # -- dense-cache attention (reference csrc/decode_attention.cu, csrc/flash_prefill.cu)
    @staticmethod
    def dense_supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
        """Whether the library serves this dense call (after the reference's own checks):
        head dim 32/64/128/256, k and v sharing strides that are multiples of 16 bytes
        (the batch stride a multiple of the position stride), 16-byte aligned pointers.
        Anything else is the PyTorch path's."""
        if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape or q.shape[-1] not in (32, 64, 128, 256):
            return False
        if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            return False
        es = q.element_size()
        sb, sh, sp, sd = k.stride()
        if v.stride() != k.stride() and not (k.shape[0] == 1 and v.stride()[1:] == k.stride()[1:]):
            return False
        if sd != 1 or sp <= 0 or sh < 0 or (sp * es) % 16 or (sh * es) % 16:
            return False
        if k.shape[0] > 1 and sb % sp:
            return False
        return all(t.data_ptr() % 16 == 0 for t in (q, k, v))

    def _dense_checks(self, name: str, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        if not (q.is_cuda and k.is_cuda and v.is_cuda):
            raise RuntimeError(f"{name}: q, k and v must be CUDA tensors")
        if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
            raise RuntimeError(f"{name}: expected B x H x L x D tensors, got q.dim()={q.dim()}")
        if name == "decode_attention" and q.shape[2] != 1:
            raise RuntimeError(
                f"decode_attention: this kernel is the L == 1 case, got a query length of "
                f"{q.shape[2]}; use flash_prefill for longer queries")
        if k.shape != v.shape:
            raise RuntimeError(f"{name}: k is {list(k.shape)} but v is {list(v.shape)}")
        if q.shape[0] != k.shape[0]:
            raise RuntimeError(f"{name}: batch mismatch, q has {q.shape[0]} and k has {k.shape[0]}")
        if q.shape[3] != k.shape[3]:
            raise RuntimeError(f"{name}: head dim mismatch, q has {q.shape[3]} and k has {k.shape[3]}")
        if k.shape[1] == 0 or q.shape[1] % k.shape[1] != 0:
            raise RuntimeError(f"{name}: H_q ({q.shape[1]}) must be a multiple of H_k ({k.shape[1]})")
        if name == "decode_attention" and k.shape[2] == 0:
            raise RuntimeError(
                "decode_attention: the cache is empty, so there is nothing to attend to; softmax "
                "over zero keys is undefined")
        if name == "flash_prefill" and not (q.shape[2] > 0 and k.shape[2] >= q.shape[2]):
            raise RuntimeError(
                f"flash_prefill: {q.shape[2]} queries against {k.shape[2]} keys; this kernel masks "
                "causally, which needs S >= L > 0")
        if q.dtype != k.dtype or q.dtype != v.dtype:
            raise RuntimeError(f"{name}: q, k and v must share a dtype, got {q.dtype}, {k.dtype} "
                               f"and {v.dtype}")
        if q.dtype == torch.float64:
            raise RuntimeError(f"{name}: float64 is not supported; the accumulators here are fp32. "
                               "Use the PyTorch path.")
        if q.stride(3) != 1 or k.stride(3) != 1 or v.stride(3) != 1:
            raise RuntimeError(f"{name}: the head dimension must be contiguous")

    def _dense(self, name: str, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               scale: float) -> torch.Tensor:
        self._dense_checks(name, q, k, v)
        b, hq, L, d = q.shape
        qt = q.transpose(1, 2)
        if not qt.is_contiguous():
            qt = qt.contiguous()
        out = torch.empty((b, L, hq, d), dtype=q.dtype, device=q.device)
        if b == 0:
            return out.transpose(1, 2)
        args = _DenseArgs(out.data_ptr(), qt.data_ptr(), k.data_ptr(), v.data_ptr(),
                          *k.stride()[:3], *v.stride()[:3], b, hq, k.shape[1], L, k.shape[2], d,
                          float(scale), DTYPE_CODES.get(q.dtype, -1))
        need = ctypes.c_uint64()
        self._check(self.lib.mvllm_dense_attention_plan(ctypes.byref(args), ctypes.byref(need)))
        ws = self.workspace(q.device, need.value)
        self._check(self.lib.mvllm_dense_attention(ctypes.byref(args), ws.data_ptr(), ws.numel(),
                                                   _stream(q.device)))
        return out.transpose(1, 2)

    def decode_attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         scale: float) -> torch.Tensor:
        """One query token per sequence against its whole dense cache (reference
        csrc/decode_attention.cu:360-435): q ``B x H_q x 1 x D``, k/v ``B x H_k x S x D``
        read through their strides. The output is ``B x H_q x 1 x D``."""
        return self._dense("decode_attention", q, k, v, scale)

    def flash_prefill(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      scale: float) -> torch.Tensor:
        """L queries against S >= L cached keys, causal with offset S - L (reference
        csrc/flash_prefill.cu:282-355). The output is ``B x H_q x L x D`` values, a
        transposed view of a token-major buffer (its ``.transpose(1, 2)`` is contiguous)."""
        return self._dense("flash_prefill", q, k, v, scale)

    def paged_attention_plan(
        self,
        num_tokens: int,
        num_seqs: int,
        num_q_heads: int,
        num_kv_heads: int,
        head_dim: int,
        block_size: int,
        max_query_len: int,
        max_context_len: int,
        q_dtype: torch.dtype,
        kv_dtype: torch.dtype,
        plan_options: dict[str, Any] | None = None,
    ) -> dict[str, int]:
        """The library's plan for a call of these sizes (``mvllm_paged_attention_plan``);
        ``plan_options`` are ``mvllm_plan_options`` fields by name."""
        plan = _Plan()
        opts = make_plan_options(plan_options)
        self._check(
            self.lib.mvllm_paged_attention_plan(
                num_tokens,
                num_seqs,
                num_q_heads,
                num_kv_heads,
                head_dim,
                block_size,
                max_query_len,
                max_context_len,
                DTYPE_CODES.get(q_dtype, -1),
                DTYPE_CODES.get(kv_dtype, -1),
                None if opts is None else ctypes.byref(opts),
                ctypes.byref(plan),
            )
        )
        out = {name: getattr(plan, name) for name, _ in _Plan._fields_}
        out["decode_mode"] = DECODE_MODES.get(out["decode_mode"], out["decode_mode"])
        return out

    def _paged_checks(self, q, key_pool, value_pool, block_tables, cu_seqlens_q, context_lens,
                      seq_lens, max_query_len, max_context_len, k_scale, v_scale,
                      strided_q: bool = False):
        """The reference's refusals for a paged call (``paged_attention.cu:608-676``) and this
        library's: raises RuntimeError; returns the contiguous metadata. ``strided_q``: q
        may have any token stride (its caller checks the rows)."""
        if not (q.is_cuda and key_pool.is_cuda and value_pool.is_cuda):
            raise RuntimeError("paged_attention: q and the pools must be CUDA tensors")
        if q.dim() != 3:
            raise RuntimeError(
                "paged_attention: expected q shaped T x H_q x D (the flattened token axis), "
                f"got {list(q.shape)}"
            )
        if key_pool.dim() != 4 or key_pool.shape != value_pool.shape:
            raise RuntimeError(
                "paged_attention: expected matching pools shaped num_blocks x P x H_k x D, got "
                f"{list(key_pool.shape)} and {list(value_pool.shape)}"
            )
        if not ((strided_q or q.is_contiguous()) and key_pool.is_contiguous()
                and value_pool.is_contiguous()):
            raise RuntimeError(
                "paged_attention: q and the pools must be contiguous; the kernel walks them by "
                "slot arithmetic rather than by stride"
            )
        fp8 = key_pool.dtype == torch.float8_e4m3fn
        if q.dtype == torch.float64:
            raise RuntimeError(
                "paged_attention: float64 is not supported; the accumulators here are fp32"
            )
        if key_pool.dtype != value_pool.dtype or (q.dtype != key_pool.dtype and not fp8):
            raise RuntimeError(
                f"paged_attention: q and the pools must share a dtype, got {q.dtype}, "
                f"{key_pool.dtype} and {value_pool.dtype}"
            )
        if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise RuntimeError(f"paged_attention: q dtype {q.dtype} is not supported")
        if q.shape[2] != key_pool.shape[3]:
            raise RuntimeError(
                f"paged_attention: head dim mismatch, q has {q.shape[2]} and the pool has "
                f"{key_pool.shape[3]}"
            )
        num_blocks, block_size, num_kv_heads, head_dim = key_pool.shape
        if num_kv_heads == 0 or q.shape[1] % num_kv_heads != 0:
            raise RuntimeError(
                f"paged_attention: H_q ({q.shape[1]}) must be a multiple of H_k ({num_kv_heads})"
            )
        if block_size <= 0 or block_size & (block_size - 1):
            raise RuntimeError(
                f"paged_attention: the block size must be a power of two, got {block_size}"
            )
        num_sequences = seq_lens.shape[0]
        if block_tables.dim() != 2 or block_tables.shape[0] != num_sequences:
            raise RuntimeError(
                f"paged_attention: expected a block table per sequence, got "
                f"{list(block_tables.shape)} for {num_sequences} sequences"
            )
        if context_lens.shape[0] != num_sequences or cu_seqlens_q.shape[0] != num_sequences + 1:
            raise RuntimeError("paged_attention: metadata disagrees on the sequence count")
        if any(
            t.dtype != torch.int32 for t in (block_tables, cu_seqlens_q, context_lens, seq_lens)
        ):
            raise RuntimeError("paged_attention: the metadata tensors must be int32")
        if not block_tables.is_contiguous():
            raise RuntimeError("paged_attention: block_tables must be contiguous")
        if not all(
            t.is_cuda and t.device == q.device
            for t in (key_pool, value_pool, block_tables, cu_seqlens_q, context_lens, seq_lens)
        ):
            raise RuntimeError("paged_attention: every tensor must be on q's CUDA device")
        if max_query_len < 1:
            raise RuntimeError(f"paged_attention: max_query_len must be >= 1, got {max_query_len}")
        if max_context_len < max_query_len:
            raise RuntimeError(
                f"paged_attention: max_context_len ({max_context_len}) must be at least "
                f"max_query_len ({max_query_len}); a pass cannot compute more tokens than it "
                "may attend over"
            )
        if fp8:
            if k_scale is None or v_scale is None:
                raise RuntimeError(
                    "paged_attention: a float8_e4m3fn pool needs k_scale and v_scale "
                    "(num_blocks x H_k float32)"
                )
            for name, s in (("k_scale", k_scale), ("v_scale", v_scale)):
                if (
                    s.dtype != torch.float32
                    or tuple(s.shape) != (num_blocks, num_kv_heads)
                    or not s.is_contiguous()
                    or s.device != q.device
                ):
                    raise RuntimeError(
                        f"paged_attention: {name} must be a contiguous float32 "
                        f"{num_blocks} x {num_kv_heads} tensor on q's device"
                    )
        elif k_scale is not None or v_scale is not None:
            raise RuntimeError("paged_attention: k_scale/v_scale apply only to a float8 pool")

        # Make sure the metadata is readable by index arithmetic.
        cu_seqlens_q = cu_seqlens_q.contiguous()
        context_lens = context_lens.contiguous()
        seq_lens = seq_lens.contiguous()
        return cu_seqlens_q, context_lens, seq_lens

    def paged_attention(
        self,
        q: torch.Tensor,
        key_pool: torch.Tensor,
        value_pool: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        context_lens: torch.Tensor,
        seq_lens: torch.Tensor,
        max_query_len: int,
        max_context_len: int,
        scale: float,
        k_scale: torch.Tensor | None = None,
        v_scale: torch.Tensor | None = None,
        out: torch.Tensor | None = None,
        plan_options: dict[str, Any] | None = None,
    ) -> torch.Tensor:
        """Ragged decode + prefill over a paged cache (reference csrc/paged_attention.cu:598-711).

        Same positional arguments and refusals as the reference. Additions, all optional:
        ``k_scale``/``v_scale`` (``num_blocks x H_k`` fp32) for a float8_e4m3fn pool,
        ``out`` to write into a caller-owned ``T x H_q x D`` tensor, and ``plan_options``
        (``mvllm_plan_options`` fields by name) to force a schedule.
        """
        cu_seqlens_q, context_lens, seq_lens = self._paged_checks(
            q, key_pool, value_pool, block_tables, cu_seqlens_q, context_lens, seq_lens,
            max_query_len, max_context_len, k_scale, v_scale)
        fp8 = key_pool.dtype == torch.float8_e4m3fn
        num_blocks, block_size, num_kv_heads, head_dim = key_pool.shape
        num_sequences = seq_lens.shape[0]

        if out is None:
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
            raise RuntimeError("paged_attention: out must be a contiguous tensor shaped like q")
        num_tokens, num_q_heads, _ = q.shape
        if num_tokens == 0 or num_sequences == 0:
            return out

        q_code = DTYPE_CODES[q.dtype]
        kv_code = DTYPE_CODES[key_pool.dtype]
        opts = make_plan_options(plan_options)
        opts_ref = None if opts is None else ctypes.byref(opts)
        plan = _Plan()
        self._check(
            self.lib.mvllm_paged_attention_plan(
                num_tokens,
                num_sequences,
                num_q_heads,
                num_kv_heads,
                head_dim,
                block_size,
                int(max_query_len),
                int(max_context_len),
                q_code,
                kv_code,
                opts_ref,
                ctypes.byref(plan),
            )
        )
        workspace = None
        if plan.workspace_bytes:
            workspace = self.workspace(q.device, plan.workspace_bytes)
        self._check(
            self.lib.mvllm_paged_attention(
                out.data_ptr(),
                q.data_ptr(),
                key_pool.data_ptr(),
                value_pool.data_ptr(),
                _ptr(k_scale),
                _ptr(v_scale),
                block_tables.data_ptr(),
                cu_seqlens_q.data_ptr(),
                context_lens.data_ptr(),
                seq_lens.data_ptr(),
                num_tokens,
                num_sequences,
                num_q_heads,
                num_kv_heads,
                head_dim,
                block_size,
                num_blocks,
                block_tables.shape[1],
                int(max_query_len),
                int(max_context_len),
                float(scale),
                q_code,
                kv_code,
                opts_ref,
                _ptr(workspace),
                0 if workspace is None else workspace.numel(),
                _stream(q.device),
            )
        )
        return out

    @staticmethod
    def paged_decode_qk_norm_rope_supported(q: torch.Tensor, key_pool: torch.Tensor,
                                            num_seqs: int) -> bool:
        """Whether ``paged_decode_qk_norm_rope`` serves a decode-only batch of this shape
        without options: a float16 or bfloat16 pool of q's dtype, head dim 128, a stream
        plan (at most 4096 sequences, at most 8 wave units of (kv head, query-head
        chunk)). The caller otherwise makes the two calls it fuses."""
        if q.dtype not in (torch.float16, torch.bfloat16) or key_pool.dtype != q.dtype:
            return False
        if key_pool.dim() != 4 or key_pool.shape[3] != 128 or q.shape[-1] != 128:
            return False
        hk = key_pool.shape[2]
        hq = q.shape[-2]
        if hk <= 0 or hq % hk:
            return False
        group = hq // hk
        chunk = 4 if group % 4 == 0 else (2 if group % 2 == 0 else 1)
        return 0 < num_seqs <= 4096 and hk * (group // chunk) <= 8

    def paged_decode_qk_norm_rope(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        q_weight: torch.Tensor,
        k_weight: torch.Tensor,
        cos: torch.Tensor,
        sin: torch.Tensor,
        eps: float,
        key_pool: torch.Tensor,
        value_pool: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        context_lens: torch.Tensor,
        seq_lens: torch.Tensor,
        max_context_len: int,
        scale: float,
        out: torch.Tensor | None = None,
        plan_options: dict[str, Any] | None = None,
    ) -> torch.Tensor:
        """A decode step's attention with its new token's QK-norm, RoPE and KV write in
        the same launch (``mvllm_paged_decode_qk_norm_rope``): bitwise
        ``qk_norm_rope_kv_write`` (positions ``context_lens - 1``, slots from the block
        tables) then ``paged_attention`` of the rotated q. q (raw, ``S x H_q x D``), k
        and v (``S x H_k x D``) may be column views of the fused projection's output;
        every sequence computes one token (``S`` rows)."""
        name = "paged_decode_qk_norm_rope"
        self._qk_norm_rope_checks(name, q, k, q_weight, k_weight, context_lens, cos, sin)
        cu_seqlens_q, context_lens, seq_lens = self._paged_checks(
            q, key_pool, value_pool, block_tables, cu_seqlens_q, context_lens, seq_lens,
            1, max_context_len, None, None, strided_q=True)
        num_blocks, block_size, num_kv_heads, head_dim = key_pool.shape
        num_seqs = seq_lens.shape[0]
        if q.shape[0] != num_seqs or v.shape != k.shape or v.dtype != q.dtype or not v.is_cuda:
            raise RuntimeError(
                f"{name}: one token per sequence: q must be {num_seqs} x H_q x D and v shaped "
                f"like k, got {tuple(q.shape)}, {tuple(k.shape)} and {tuple(v.shape)}")
        if not self.paged_decode_qk_norm_rope_supported(q, key_pool, num_seqs):
            raise RuntimeError(f"{name}: this dtype / head dim / batch is not served")
        d = head_dim

        def rows_ok(t):  # heads contiguous within each token
            return t.stride(2) == 1 and t.stride(1) == d
        if not (rows_ok(q) and rows_ok(k) and rows_ok(v)) or k.stride(0) != v.stride(0):
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        if out is None:
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
            raise RuntimeError(f"{name}: out must be a contiguous tensor shaped like q")
        if num_seqs == 0:
            return out
        code = DTYPE_CODES[q.dtype]
        num_q_heads = q.shape[1]
        opts = make_plan_options(plan_options)
        opts_ref = None if opts is None else ctypes.byref(opts)
        plan = _Plan()
        self._check(self.lib.mvllm_paged_attention_plan(
            num_seqs, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, 1,
            int(max_context_len), code, code, opts_ref, ctypes.byref(plan)))
        workspace = self.workspace(q.device, max(int(plan.workspace_bytes), 256))
        self._check(self.lib.mvllm_paged_decode_qk_norm_rope(
            out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), q.stride(0), k.stride(0),
            q_weight.contiguous().data_ptr(), k_weight.contiguous().data_ptr(),
            cos.contiguous().data_ptr(), sin.contiguous().data_ptr(), cos.shape[0], float(eps),
            key_pool.data_ptr(), value_pool.data_ptr(), block_tables.data_ptr(),
            cu_seqlens_q.data_ptr(), context_lens.data_ptr(), seq_lens.data_ptr(), num_seqs,
            num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, block_tables.shape[1],
            int(max_context_len), float(scale), code, opts_ref, workspace.data_ptr(),
            workspace.numel(), _stream(q.device)))
        return out


def load_extension(verbose: bool = False) -> HipExtension:
    """Return the bound library, building it first only if nothing is built yet.

    Raises :class:`ToolchainError` when no GPU is visible: there is no CPU
    implementation behind this object, by design.
    """
    global _extension
    with _lock:
        if _extension is not None:
            return _extension
        if not torch.cuda.is_available():
            raise ToolchainError("no GPU visible; the HIP kernels need an MI355X (gfx950)")
        if not LIB_PATH.exists():
            build_library(verbose=verbose)
        _extension = HipExtension(open_library())
        return _extension


def rebuild(verbose: bool = True) -> HipExtension:
    """Compile from scratch and rebind (only valid before the old library was used)."""
    global _extension
    with _lock:
        _extension = None
    build_library(verbose=verbose)
    return load_extension(verbose=verbose)


def toolchain_report() -> dict[str, Any]:
    report: dict[str, Any] = {
        "python": sys.version.split()[0],
        "torch": torch.__version__,
        "torch_hip": getattr(torch.version, "hip", None),
        "hipcc": HIPCC,
        "arch": ARCH,
        "library": str(LIB_PATH),
        "library_built": LIB_PATH.exists(),
        "sources": [p.name for p in sources()],
        "gpu_available": torch.cuda.is_available(),
    }
    if torch.cuda.is_available():
        props = torch.cuda.get_device_properties(0)
        report["gpu"] = props.name
        report["gcn_arch"] = getattr(props, "gcnArchName", None)
        report["compute_units"] = props.multi_processor_count
        report["vram_gb"] = round(props.total_memory / 1024**3, 2)
    return report


def main() -> int:
    import argparse

    parser = argparse.ArgumentParser(description="Build the Mini-vLLM MI355X kernel library.")
    parser.add_argument("--build", action="store_true", help="compile before anything else")
    args = parser.parse_args()
    if args.build:
        build_library(verbose=True)
    for key, value in toolchain_report().items():
        print(f"{key:>16}: {value}")
    if not torch.cuda.is_available():
        return 0
    ext = load_extension(verbose=True)
    x = torch.randn(1024, device="cuda")
    ok = torch.allclose(ext.hello(x, 2.0, 3.0), 2.0 * x + 3.0)
    print(f"\nhello(x, 2, 3) == 2x + 3 : {'ok' if ok else 'MISMATCH'}")
    return 0 if ok else 1


if __name__ == "__main__":
    raise SystemExit(main())
