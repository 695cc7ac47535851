"""kernelfoundry_amd -- MI355X (gfx950) flash-attention forward.

Python host side over the C ABI of ``lib/libkf_attn.so`` (include/kf/attn.h).
The compute runs only in the HIP kernels of that library; there is no CPU or
PyTorch fallback: if the library is missing, every entry point raises.

Interface, mirroring the reference harness (sviraaj/kernelfoundry):

* ``launch_flash_attn(Q, K, V, O, B, S, H_q, H_kv, D, stream=0)`` -- the
  reference launcher (tests/test_flash_attn.cu:52-113) on raw device
  pointers: q_len = kv_len = S, synchronous, returns a hipError_t value
  (0 on success, hipErrorInvalidValue = 1 for an unsupported D or shape).
* ``attn_fwd(Q, K, V, ...)`` -- asynchronous forward on torch device tensors
  (torch provides device memory and the stream; it is plumbing only), with
  separate q_len / kv_len (decode) and optional Mi / Li outputs, as the
  bench's ``launch_once`` (tests/bench_flash_attn.cu:39-54).
* ``attn_fwd_ptr(...)`` -- the same on raw pointers, returning the kf status.
* ``attn_fwd(..., causal=True, kv_lens=...)`` / ``attn_fwd_ex_ptr(...)`` --
  kf_attn_fwd_ex: bottom-right-aligned causal masking and per-sequence key
  counts over a pre-allocated K/V cache (no reference counterpart).
* ``attn_decode_paged(Q, K_pages, V_pages, block_table, kv_lens, ...)`` --
  kf_attn_decode_paged: decode over a paged K/V cache (page pools
  [num_pages, H_kv, page_size, D] and a per-sequence block table).
* ``plan(B, q_len, kv_len, H_q, H_kv, D, num_cus=None)`` -- which kernels run,
  sized for the current device's compute units (or ``num_cus``).
"""
from __future__ import annotations

import ctypes
import os
import re
from dataclasses import dataclass

__all__ = [
    "KfError", "LIB_PATH", "load_library", "plan", "workspace_bytes", "attn_fwd",
    "attn_fwd_ptr", "launch_flash_attn", "status_string", "exported_symbols",
    "KF_OK", "KF_ERR_HEAD_DIM", "KF_ERR_GQA", "KF_ERR_SIZE", "KF_ERR_NULL",
    "KF_ERR_WORKSPACE", "KF_ERR_ALIGN", "KF_ERR_HIP", "KF_ERR_FLAGS", "KF_ERR_SCRATCH",
    "KF_ATTN_CAUSAL",
    "KF_ATTN_OUT_F16", "KF_ATTN_OUT_BF16", "KF_ATTN_LSE",
    "PATH_NAMES", "attn_fwd_ex_ptr", "attn_decode_paged", "attn_decode_paged_ptr",
    "paged_workspace_bytes", "kernel_names",
]

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libkf_attn.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG), "include", "kf", "attn.h")

KF_OK = 0
KF_ERR_HEAD_DIM = 1
KF_ERR_GQA = 2
KF_ERR_SIZE = 3
KF_ERR_NULL = 4
KF_ERR_WORKSPACE = 5
KF_ERR_ALIGN = 6
KF_ERR_HIP = 7
KF_ERR_FLAGS = 8
KF_ERR_SCRATCH = 9
KF_ATTN_CAUSAL = 1
KF_ATTN_OUT_F16 = 2
KF_ATTN_OUT_BF16 = 4
KF_ATTN_LSE = 8

PATH_NAMES = {0: "prefill", 1: "decode", 2: "decode_split", 3: "prefill_split"}

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1


class KfError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"kf status {status}: {message}")
        self.status = status


class _PlanStruct(ctypes.Structure):
    _fields_ = [
        ("path", ctypes.c_int),
        ("rows_per_group", ctypes.c_int),
        ("num_splits", ctypes.c_int),
        ("kv_per_split", ctypes.c_int),
        ("grid_blocks", ctypes.c_int),
        ("block_threads", ctypes.c_int),
        ("workspace_bytes", ctypes.c_size_t),
        ("splits_per_block", ctypes.c_int),
    ]


@dataclass(frozen=True)
class Plan:
    path: str
    rows_per_group: int
    num_splits: int
    kv_per_split: int
    grid_blocks: int
    block_threads: int
    workspace_bytes: int
    splits_per_block: int = 0


_lib = None


def _bind_torch_hip_runtime():
    """Load torch's HIP runtime before libkf_attn.so, if torch is installed.

    PyTorch-ROCm wheels ship their own libamdhip64 / libhsa-runtime64, which
    torch loads by the unversioned name; libkf_attn.so asks for
    libamdhip64.so.7 (soname of both copies).  Loaded after torch, the
    library binds to torch's runtime by soname.  Loaded before torch, it pulls
    in the system runtime and torch then adds its own: two HIP and two HSA
    runtimes in one process, torch's tensors and streams living in the one
    and this library's launches in the other (seen as failed launches and
    crashes).  Importing torch first keeps one runtime.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load_library(path: str = LIB_PATH):
    """Load libkf_attn.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m kernelfoundry_amd.build` "
            "(or __graft_entry__.build()); there is no fallback implementation")
    _bind_torch_hip_runtime()
    lib = ctypes.CDLL(path)
    i, p, sz = ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
    lib.kf_attn_plan.argtypes = [i] * 6 + [ctypes.POINTER(_PlanStruct)]
    lib.kf_attn_plan.restype = i
    lib.kf_attn_plan_for_cus.argtypes = [i] * 7 + [ctypes.POINTER(_PlanStruct)]
    lib.kf_attn_plan_for_cus.restype = i
    lib.kf_attn_workspace_bytes.argtypes = [i] * 6
    lib.kf_attn_workspace_bytes.restype = sz
    lib.kf_attn_kernel_names.argtypes = [i] * 7 + [p, ctypes.c_char_p, sz]
    lib.kf_attn_kernel_names.restype = i
    lib.kf_attn_fwd.argtypes = [p, p, p, p, p, p] + [i] * 6 + [p, sz, p]
    lib.kf_attn_fwd.restype = i
    lib.kf_attn_fwd_ex.argtypes = [p, p, p, p, p, p] + [i] * 6 + [p, i, p, sz, p]
    lib.kf_attn_fwd_ex.restype = i
    lib.kf_attn_fwd_noalloc.argtypes = [p, p, p, p, p, p] + [i] * 6 + [p, i, p]
    lib.kf_attn_fwd_noalloc.restype = i
    lib.kf_attn_noalloc_scratch_bytes.argtypes = []
    lib.kf_attn_noalloc_scratch_bytes.restype = sz
    lib.kf_attn_decode_paged.argtypes = [p] * 8 + [i] * 9 + [p, sz, p]
    lib.kf_attn_decode_paged.restype = i
    lib.kf_attn_decode_paged_workspace_bytes.argtypes = [i] * 7
    lib.kf_attn_decode_paged_workspace_bytes.restype = sz
    lib.kf_launch_flash_attn.argtypes = [p, p, p, p] + [i] * 5 + [p]
    lib.kf_launch_flash_attn.restype = i
    lib.kf_status_string.argtypes = [i]
    lib.kf_status_string.restype = ctypes.c_char_p
    lib.kf_last_hip_error.argtypes = []
    lib.kf_last_hip_error.restype = i
    lib.kf_version.argtypes = []
    lib.kf_version.restype = ctypes.c_char_p
    _lib = lib
    return lib


def exported_symbols(header: str = HEADER_PATH):
    """Names of the functions declared in include/kf/attn.h."""
    text = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(kf_\w+)\s*\(", text, re.M)))


def status_string(status: int) -> str:
    return load_library().kf_status_string(int(status)).decode()


def plan(B, q_len, kv_len, H_q, H_kv, D, num_cus=None) -> Plan:
    """The dispatch for the current device (kf_attn_plan), or for a device
    with ``num_cus`` compute units (kf_attn_plan_for_cus)."""
    out = _PlanStruct()
    lib = load_library()
    if num_cus is None:
        st = lib.kf_attn_plan(B, q_len, kv_len, H_q, H_kv, D, ctypes.byref(out))
    else:
        st = lib.kf_attn_plan_for_cus(B, q_len, kv_len, H_q, H_kv, D, int(num_cus),
                                      ctypes.byref(out))
    if st != KF_OK:
        raise KfError(st, status_string(st))
    return Plan(PATH_NAMES[out.path], out.rows_per_group, out.num_splits, out.kv_per_split,
                out.grid_blocks, out.block_threads, int(out.workspace_bytes), out.splits_per_block)


def kernel_names(B, q_len, kv_len, H_q, H_kv, D, causal=False, masked=False) -> str:
    """The kernels kf_attn_fwd_ex runs for this shape on the current device,
    as a profiler names them (``masked``: a kv_lens array is passed)."""
    buf = ctypes.create_string_buffer(256)
    st = load_library().kf_attn_kernel_names(B, q_len, kv_len, H_q, H_kv, D,
                                             KF_ATTN_CAUSAL if causal else 0,
                                             1 if masked else None, buf, len(buf))
    if st != KF_OK:
        raise KfError(st, status_string(st))
    return buf.value.decode()


def workspace_bytes(B, q_len, kv_len, H_q, H_kv, D) -> int:
    return int(load_library().kf_attn_workspace_bytes(B, q_len, kv_len, H_q, H_kv, D))


def attn_fwd_ptr(Q, K, V, O, Mi, Li, B, q_len, kv_len, H_q, H_kv, D, workspace=0,
                 workspace_bytes=0, stream=0) -> int:
    """kf_attn_fwd on raw device addresses (ints); returns the kf status."""
    return int(load_library().kf_attn_fwd(Q, K, V, O, Mi or None, Li or None, B, q_len, kv_len,
                                          H_q, H_kv, D, workspace or None, workspace_bytes,
                                          stream or None))


def attn_fwd_ex_ptr(Q, K, V, O, Mi, Li, B, q_len, kv_len, H_q, H_kv, D, kv_lens=0, flags=0,
                    workspace=0, workspace_bytes=0, stream=0) -> int:
    """kf_attn_fwd_ex on raw device addresses (ints); returns the kf status."""
    return int(load_library().kf_attn_fwd_ex(Q, K, V, O, Mi or None, Li or None, B, q_len,
                                             kv_len, H_q, H_kv, D, kv_lens or None, flags,
                                             workspace or None, workspace_bytes, stream or None))


def paged_workspace_bytes(B, q_len, H_q, H_kv, D, page_size, max_pages_per_seq) -> int:
    return int(load_library().kf_attn_decode_paged_workspace_bytes(B, q_len, H_q, H_kv, D,
                                                                    page_size, max_pages_per_seq))


def attn_decode_paged_ptr(Q, K_pages, V_pages, block_table, kv_lens, O, Mi, Li, B, q_len, H_q,
                          H_kv, D, page_size, max_pages_per_seq, num_pages, flags=0, workspace=0,
                          workspace_bytes=0, stream=0) -> int:
    """kf_attn_decode_paged on raw device addresses (ints); returns the kf status."""
    return int(load_library().kf_attn_decode_paged(
        Q, K_pages, V_pages, block_table or None, kv_lens or None, O, Mi or None, Li or None,
        B, q_len, H_q, H_kv, D, page_size, max_pages_per_seq, num_pages, flags,
        workspace or None, workspace_bytes, stream or None))


def launch_flash_attn(Q, K, V, O, B, S, H_q, H_kv, D, stream=0) -> int:
    """Reference launcher contract on raw device addresses; returns hipError_t."""
    return int(load_library().kf_launch_flash_attn(Q, K, V, O, B, S, H_q, H_kv, D, stream or None))


def _out_flags(torch, out_dtype, return_lse):
    f = {None: 0, torch.float32: 0, torch.float16: KF_ATTN_OUT_F16,
         torch.bfloat16: KF_ATTN_OUT_BF16}
    if out_dtype not in f:
        raise ValueError("out_dtype must be float32, float16 or bfloat16")
    return f[out_dtype] | (KF_ATTN_LSE if return_lse else 0)


def _new(torch, shape, dtype, device, stream):
    """A new tensor written on ``stream``, allocated from ``stream``'s pool of
    torch's caching allocator.  A block of that pool was last used by work on
    ``stream`` itself, so the launch that follows on ``stream`` is ordered
    after that work; a block taken from another stream's pool (torch's
    current one) could still be in use by a kernel queued there.  Freed, the
    tensor returns to ``stream``'s pool, so it is not reused before the
    launch on ``stream`` has finished with it."""
    with torch.cuda.stream(stream):
        return torch.empty(shape, dtype=dtype, device=device)


def _output(torch, out, shape, out_dtype, device, stream):
    """The output tensor: a new one, or the caller's after checking that the
    kernel's writes (shape x element size of ``out_dtype``) land inside it."""
    dtype = out_dtype or torch.float32
    if out is None:
        return _new(torch, shape, dtype, device, stream)
    if out.dtype != dtype or tuple(out.shape) != tuple(shape) or out.device != device \
            or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {dtype} tensor of shape {tuple(shape)} "
                         f"on {device}")
    return out


def _workspace(torch, workspace, need, device, stream):
    """The split-KV workspace: the caller's if it is a large enough buffer on
    the device, else a new one (kept alive until ``stream`` passes it)."""
    if not need:
        return None
    if workspace is not None:
        if workspace.device != device or not workspace.is_contiguous():
            raise ValueError(f"workspace must be a contiguous tensor on {device}")
        if workspace.numel() * workspace.element_size() >= need:
            return workspace
    return _new(torch, need, torch.uint8, device, stream)


def attn_fwd(Q, K, V, out=None, *, return_stats=False, workspace=None, stream=None,
             causal=False, kv_lens=None, out_dtype=None, return_lse=False):
    """Attention forward on torch tensors resident on the GPU.

    Q [B, H_q, q_len, D] fp16, K/V [B, H_kv, kv_len, D] fp16, contiguous.
    Returns O [B, H_q, q_len, D] (fp32, or ``out_dtype`` fp16 / bf16), or
    (O, Mi, Li) with ``return_stats``, or (O, LSE) with ``return_lse``.
    Asynchronous on ``stream`` (default: torch's current stream).
    ``causal`` / ``kv_lens`` (int32 GPU tensor [B]) select kf_attn_fwd_ex.
    """
    import torch

    if return_stats and return_lse:
        raise ValueError("return_stats and return_lse are exclusive")
    flags = _out_flags(torch, out_dtype, return_lse)

    if Q.dtype != torch.float16 or K.dtype != torch.float16 or V.dtype != torch.float16:
        raise TypeError("Q, K, V must be float16")
    if not (Q.is_cuda and K.is_cuda and V.is_cuda):
        raise ValueError("Q, K, V must be GPU tensors")
    if not (Q.is_contiguous() and K.is_contiguous() and V.is_contiguous()):
        raise ValueError("Q, K, V must be contiguous [B, H, S, D]")
    if Q.dim() != 4 or K.dim() != 4 or K.shape != V.shape:
        raise ValueError("expected Q [B,H_q,q_len,D] and K, V [B,H_kv,kv_len,D]")
    if K.device != Q.device or V.device != Q.device:
        raise ValueError("Q, K, V must be on one device")
    B, H_q, q_len, D = Q.shape
    Bk, H_kv, kv_len, Dk = K.shape
    if Bk != B or Dk != D:
        raise ValueError("Q and K/V disagree on B or D")
    if stream is None:
        stream = torch.cuda.current_stream(Q.device)
    out = _output(torch, out, (B, H_q, q_len, D), out_dtype, Q.device, stream)
    Mi = Li = None
    if return_stats or return_lse:
        Mi = _new(torch, (B, H_q, q_len), torch.float32, Q.device, stream)
    if return_stats:
        Li = _new(torch, (B, H_q, q_len), torch.float32, Q.device, stream)
    need = workspace_bytes(B, q_len, kv_len, H_q, H_kv, D)
    workspace = _workspace(torch, workspace, need, Q.device, stream)
    if kv_lens is not None:
        # A contiguous copy would be made on torch's current stream, unordered
        # with a launch on another ``stream``: require the caller's layout.
        if kv_lens.dtype != torch.int32 or kv_lens.device != Q.device or kv_lens.numel() != B \
                or not kv_lens.is_contiguous():
            raise ValueError("kv_lens must be a contiguous int32 tensor of B elements on "
                             "Q's device")
    st = attn_fwd_ex_ptr(Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr(),
                         Mi.data_ptr() if Mi is not None else 0,
                         Li.data_ptr() if Li is not None else 0,
                         B, q_len, kv_len, H_q, H_kv, D,
                         kv_lens.data_ptr() if kv_lens is not None else 0,
                         (KF_ATTN_CAUSAL if causal else 0) | flags,
                         workspace.data_ptr() if workspace is not None else 0,
                         need, stream.cuda_stream)
    if st != KF_OK:
        msg = status_string(st)
        if st == KF_ERR_HIP:
            msg += f" (hipError_t {load_library().kf_last_hip_error()})"
        raise KfError(st, msg)
    if return_lse:
        return out, Mi
    return (out, Mi, Li) if return_stats else out


def attn_decode_paged(Q, K_pages, V_pages, block_table, kv_lens, out=None, *, return_stats=False,
                      causal=False, workspace=None, stream=None, out_dtype=None,
                      return_lse=False):
    """Decode over a paged K/V cache on torch GPU tensors.

    Q [B, H_q, q_len, D] fp16; K_pages / V_pages [num_pages, H_kv, page_size,
    D] fp16; block_table int32 [B, max_pages_per_seq]; kv_lens int32 [B].
    Returns O [B, H_q, q_len, D] fp32 (and Mi, Li with ``return_stats``).
    """
    import torch

    if return_stats and return_lse:
        raise ValueError("return_stats and return_lse are exclusive")
    flags = _out_flags(torch, out_dtype, return_lse)
    for t, name in ((Q, "Q"), (K_pages, "K_pages"), (V_pages, "V_pages")):
        if t.dtype != torch.float16 or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float16 GPU tensor")
    for t, name in ((block_table, "block_table"), (kv_lens, "kv_lens")):
        if t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 GPU tensor")
    if any(t.device != Q.device for t in (K_pages, V_pages, block_table, kv_lens)):
        raise ValueError("all tensors must be on Q's device")
    if Q.dim() != 4 or K_pages.dim() != 4:
        raise ValueError("expected Q [B,H_q,q_len,D] and K/V pages [num_pages,H_kv,page_size,D]")
    B, H_q, q_len, D = Q.shape
    num_pages, H_kv, page_size, Dk = K_pages.shape
    if K_pages.shape != V_pages.shape or Dk != D:
        raise ValueError("K_pages / V_pages must be [num_pages, H_kv, page_size, D]")
    if block_table.dim() != 2 or block_table.shape[0] != B or kv_lens.numel() != B:
        raise ValueError("block_table must be [B, max_pages_per_seq] and kv_lens [B]")
    max_pages = block_table.shape[1]
    if stream is None:
        stream = torch.cuda.current_stream(Q.device)
    out = _output(torch, out, (B, H_q, q_len, D), out_dtype, Q.device, stream)
    Mi = Li = None
    if return_stats or return_lse:
        Mi = _new(torch, (B, H_q, q_len), torch.float32, Q.device, stream)
    if return_stats:
        Li = _new(torch, (B, H_q, q_len), torch.float32, Q.device, stream)
    need = paged_workspace_bytes(B, q_len, H_q, H_kv, D, page_size, max_pages)
    workspace = _workspace(torch, workspace, need, Q.device, stream)
    st = attn_decode_paged_ptr(Q.data_ptr(), K_pages.data_ptr(), V_pages.data_ptr(),
                               block_table.data_ptr(), kv_lens.data_ptr(), out.data_ptr(),
                               Mi.data_ptr() if Mi is not None else 0,
                               Li.data_ptr() if Li is not None else 0,
                               B, q_len, H_q, H_kv, D, page_size, max_pages, num_pages,
                               (KF_ATTN_CAUSAL if causal else 0) | flags,
                               workspace.data_ptr() if workspace is not None else 0,
                               need, stream.cuda_stream)
    if st != KF_OK:
        msg = status_string(st)
        if st == KF_ERR_HIP:
            msg += f" (hipError_t {load_library().kf_last_hip_error()})"
        raise KfError(st, msg)
    if return_lse:
        return out, Mi
    return (out, Mi, Li) if return_stats else out
