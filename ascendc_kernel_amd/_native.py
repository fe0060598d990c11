"""ctypes binding of ``libdsa_mi355x.so`` (declared in ``include/dsa_abi.h``).

The library is the only compute path: if it is missing, cannot be loaded, or a
tensor is not on a HIP device, these functions raise instead of computing
anything another way.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

from . import build as _build

ABI_VERSION = 2

DSA_SA_AUTO = 0
DSA_SA_MULTIPLICITY = 1
DSA_SA_GATHER = 2

DSA_ROPE_CPU = 0
DSA_ROPE_TORCH_ROCM = 1

EXPORTS = (
    "dsa_abi_version",
    "dsa_strerror",
    "dsa_sparse_attn_fwd",
    "dsa_sparse_attn_fwd_i64",
    "dsa_sparse_mla_fwd",
    "dsa_sparse_mla_fwd_i64",
    "dsa_sparse_mla_workspace_bytes",
    "dsa_sparse_mla_fwd_ws",
    "dsa_sparse_mla_fwd_i64_ws",
    "dsa_indexer_rope",
    "dsa_indexer_score_topk",
    "dsa_indexer_workspace_bytes",
    "dsa_indexer_score_topk_ws",
    "dsa_indexer_score_topk_noalloc",
    "dsa_indexer_scores",
    "dsa_indexer_q_proj",
)

_c_i64 = ctypes.c_int64
_c_vp = ctypes.c_void_p
_lib: Optional[ctypes.CDLL] = None


class DsaError(RuntimeError):
    """A non-zero status returned by the C ABI."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed: {msg} (code {code})")
        self.code = code


def lib_path() -> str:
    return os.environ.get("DSA_MI355X_LIB", _build.LIB_PATH)


def load() -> ctypes.CDLL:
    """Load the library once; raises RuntimeError when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m ascendc_kernel_amd.build` "
            "(there is no other implementation of these operators)")
    lib = ctypes.CDLL(path)
    lib.dsa_abi_version.restype = ctypes.c_int
    lib.dsa_abi_version.argtypes = []
    lib.dsa_strerror.restype = ctypes.c_char_p
    lib.dsa_strerror.argtypes = [ctypes.c_int]
    for name in ("dsa_sparse_attn_fwd", "dsa_sparse_attn_fwd_i64"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [
            _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
            ctypes.c_float, ctypes.c_int32, _c_vp]
    for name in ("dsa_sparse_mla_fwd", "dsa_sparse_mla_fwd_i64"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [
            _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
            ctypes.c_float, _c_vp]
    for name in ("dsa_sparse_mla_fwd_ws", "dsa_sparse_mla_fwd_i64_ws"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [
            _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
            ctypes.c_float, _c_vp, _c_i64, _c_vp]
    lib.dsa_sparse_mla_workspace_bytes.restype = ctypes.c_int64
    lib.dsa_sparse_mla_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64]
    lib.dsa_indexer_rope.restype = ctypes.c_int
    lib.dsa_indexer_rope.argtypes = [
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int32, _c_vp]
    lib.dsa_indexer_score_topk.restype = ctypes.c_int
    lib.dsa_indexer_score_topk.argtypes = [
        _c_vp, _c_vp, _c_i64, _c_vp, ctypes.c_float, _c_vp, ctypes.c_int32, _c_vp,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        ctypes.c_int32, _c_i64, _c_vp]
    lib.dsa_indexer_workspace_bytes.restype = ctypes.c_int64
    lib.dsa_indexer_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]
    lib.dsa_indexer_score_topk_ws.restype = ctypes.c_int
    lib.dsa_indexer_score_topk_ws.argtypes = [
        _c_vp, _c_vp, _c_i64, _c_vp, ctypes.c_float, _c_vp, ctypes.c_int32, _c_vp,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        ctypes.c_int32, _c_i64, _c_vp, _c_i64, _c_vp]
    lib.dsa_indexer_score_topk_noalloc.restype = ctypes.c_int
    lib.dsa_indexer_score_topk_noalloc.argtypes = [
        _c_vp, _c_vp, _c_i64, _c_vp, ctypes.c_float, _c_vp, ctypes.c_int32, _c_vp,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        ctypes.c_int32, _c_i64, _c_vp]
    lib.dsa_indexer_scores.restype = ctypes.c_int
    lib.dsa_indexer_scores.argtypes = [
        _c_vp, _c_vp, _c_i64, _c_vp, ctypes.c_float, _c_vp, ctypes.c_int32, _c_vp,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int32, _c_vp]
    lib.dsa_indexer_q_proj.restype = ctypes.c_int
    lib.dsa_indexer_q_proj.argtypes = [
        _c_vp, _c_vp, _c_vp, ctypes.c_int32, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]
    v = lib.dsa_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {v}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def _check(fn: str, code: int) -> None:
    if code != 0:
        msg = load().dsa_strerror(code).decode()
        raise DsaError(fn, code, msg)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_gpu(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError("DSA kernels run on a HIP device only; got a tensor on "
                               f"{t.device}")
        if t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def sparse_attn_fwd(q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor,
                    attn_sink: torch.Tensor, softmax_scale: float,
                    variant: int = DSA_SA_AUTO) -> torch.Tensor:
    """Task1 forward on the GPU; shapes as in reference/task1_v0_ref.py:5-24."""
    lib = load()
    if q.dim() != 4 or kv.dim() != 3 or topk_idxs.dim() != 3:
        raise ValueError("expected q [b,m,h,d], kv [b,n_kv,d], topk_idxs [b,m,topk]")
    b, m, h, d = q.shape
    if kv.shape[0] != b or kv.shape[2] != d or tuple(topk_idxs.shape[:2]) != (b, m):
        raise ValueError(f"inconsistent shapes q{tuple(q.shape)} kv{tuple(kv.shape)} "
                         f"topk_idxs{tuple(topk_idxs.shape)}")
    if q.dtype != torch.bfloat16 or kv.dtype != torch.bfloat16:
        raise TypeError("q and kv must be bfloat16")
    if topk_idxs.dtype not in (torch.int32, torch.int64):
        raise TypeError("topk_idxs must be int32 or int64")
    if attn_sink.numel() != h:
        raise ValueError(f"attn_sink has {attn_sink.numel()} entries, expected {h}")
    dev = _require_gpu(q, kv, topk_idxs)
    q = q.contiguous()
    kv = kv.contiguous()
    idx = topk_idxs.contiguous()  # int64 indices are read as they are (no narrowing pass)
    fn = "dsa_sparse_attn_fwd_i64" if idx.dtype == torch.int64 else "dsa_sparse_attn_fwd"
    sink = attn_sink.detach().to(device=dev, dtype=torch.float32).contiguous()
    out = torch.empty_like(q)
    rc = getattr(lib, fn)(
        q.data_ptr(), kv.data_ptr(), idx.data_ptr(), sink.data_ptr(), out.data_ptr(),
        b, m, h, d, kv.shape[1], idx.shape[2], float(softmax_scale), int(variant), _stream(q))
    _check(fn, rc)
    return out


def sparse_mla_fwd(q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor,
                   attn_sink: torch.Tensor, softmax_scale: float, v_dim: int,
                   split: bool = True) -> torch.Tensor:
    """Sparse MLA on the GPU: q [b,m,h,d_qk], kv [b,n_kv,>=d_qk]; keys are kv[..., :d_qk],
    values kv[..., :v_dim]; returns bf16 [b,m,h,v_dim]. split=False keeps the one-pass
    kernel also where the library would split the slot lists (few tokens)."""
    lib = load()
    if q.dim() != 4 or kv.dim() != 3 or topk_idxs.dim() != 3:
        raise ValueError("expected q [b,m,h,d_qk], kv [b,n_kv,kv_dim], topk_idxs [b,m,topk]")
    b, m, h, dqk = q.shape
    if kv.shape[0] != b or kv.shape[2] < dqk or tuple(topk_idxs.shape[:2]) != (b, m):
        raise ValueError(f"inconsistent shapes q{tuple(q.shape)} kv{tuple(kv.shape)} "
                         f"topk_idxs{tuple(topk_idxs.shape)}")
    if q.dtype != torch.bfloat16 or kv.dtype != torch.bfloat16:
        raise TypeError("q and kv must be bfloat16")
    if topk_idxs.dtype not in (torch.int32, torch.int64):
        raise TypeError("topk_idxs must be int32 or int64")
    if attn_sink.numel() != h:
        raise ValueError(f"attn_sink has {attn_sink.numel()} entries, expected {h}")
    dev = _require_gpu(q, kv, topk_idxs)
    q = q.contiguous()
    kv = kv.contiguous()
    idx = topk_idxs.contiguous()  # int64 indices are read as they are (no narrowing pass)
    sink = attn_sink.detach().to(device=dev, dtype=torch.float32).contiguous()
    out = torch.empty(b, m, h, v_dim, dtype=torch.bfloat16, device=dev)
    args = (q.data_ptr(), kv.data_ptr(), idx.data_ptr(), sink.data_ptr(), out.data_ptr(),
            b, m, h, dqk, v_dim, kv.shape[2], kv.shape[1], idx.shape[2], float(softmax_scale))
    # Few tokens (decode): the slot lists are split over workgroups whose partial
    # results go to a workspace from torch's caching allocator.
    ws_bytes = int(lib.dsa_sparse_mla_workspace_bytes(b, m, h, idx.shape[2])) if split else 0
    if ws_bytes < 0:
        _check("dsa_sparse_mla_workspace_bytes", ws_bytes)
    if ws_bytes > 0:
        fn = "dsa_sparse_mla_fwd_i64_ws" if idx.dtype == torch.int64 else "dsa_sparse_mla_fwd_ws"
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        rc = getattr(lib, fn)(*args, ws.data_ptr(), ws_bytes, _stream(q))
    else:
        fn = "dsa_sparse_mla_fwd_i64" if idx.dtype == torch.int64 else "dsa_sparse_mla_fwd"
        rc = getattr(lib, fn)(*args, _stream(q))
    _check(fn, rc)
    return out


def indexer_rope_(q: torch.Tensor, freqs_cis: torch.Tensor, rope_head_dim: int,
                  mode: int = DSA_ROPE_TORCH_ROCM) -> torch.Tensor:
    """In-place RoPE on q[..., -rd:] of a contiguous [b, s, h, d] bf16 tensor."""
    lib = load()
    if q.dim() != 4 or q.dtype != torch.bfloat16 or not q.is_contiguous():
        raise ValueError("q must be a contiguous bf16 [b, s, h, d] tensor")
    b, s, h, d = q.shape
    fr = _freqs_view(freqs_cis, s, rope_head_dim)
    _require_gpu(q, fr)
    rc = lib.dsa_indexer_rope(q.data_ptr(), fr.data_ptr(), b, s, h, d, rope_head_dim,
                              int(mode), _stream(q))
    _check("dsa_indexer_rope", rc)
    return q


def _freqs_view(freqs_cis: torch.Tensor, s: int, rd: int) -> torch.Tensor:
    if freqs_cis.dtype != torch.complex64:
        raise TypeError("freqs_cis must be complex64")
    fr = freqs_cis.reshape(freqs_cis.shape[0], -1)
    if fr.shape[0] < s or fr.shape[1] != rd // 2:
        raise ValueError(f"freqs_cis {tuple(freqs_cis.shape)} does not cover {s} positions x {rd // 2}")
    return torch.view_as_real(fr[:s].contiguous())


def indexer_score_topk(q: torch.Tensor, kv_cache: torch.Tensor, wl: torch.Tensor,
                       w_scale: float, freqs_cis: Optional[torch.Tensor], rope_head_dim: int,
                       n_cand: int, k_out: int, ratio: int, causal: bool, offset: int,
                       rope_mode: int = DSA_ROPE_TORCH_ROCM, use_workspace: bool = True) -> torch.Tensor:
    """Task2 score + mask + top-k; returns int64 [b, s, k_out].

    q: bf16 [b, s, h, d] (contiguous); kv_cache: bf16 [>=b, >=n_cand, d] with unit
    row stride; wl: bf16 [b, s, h]; freqs_cis: complex64 rows for the s positions.
    When the configuration takes a workspace (64 heads x 128) it is allocated from
    torch's caching allocator and passed in (use_workspace=False: the single-kernel path).
    """
    lib = load()
    b, s, h, d = q.shape
    if q.dtype != torch.bfloat16 or kv_cache.dtype != torch.bfloat16 or wl.dtype != torch.bfloat16:
        raise TypeError("q, kv_cache and wl must be bfloat16")
    if kv_cache.dim() != 3 or kv_cache.shape[0] < b or kv_cache.shape[1] < n_cand or kv_cache.shape[2] != d:
        raise ValueError(f"kv_cache {tuple(kv_cache.shape)} does not cover [{b}, {n_cand}, {d}]")
    if kv_cache.stride(2) != 1 or kv_cache.stride(1) != d:
        kv_cache = kv_cache[:b, :n_cand].contiguous()
    if tuple(wl.shape) != (b, s, h):
        raise ValueError(f"wl {tuple(wl.shape)} != {(b, s, h)}")
    q = q.contiguous()
    wl = wl.contiguous()
    fr = _freqs_view(freqs_cis, s, rope_head_dim) if freqs_cis is not None else None
    _require_gpu(q, kv_cache, wl, *([fr] if fr is not None else []))
    out = torch.empty(b, s, k_out, dtype=torch.int64, device=q.device)
    ws_bytes = int(lib.dsa_indexer_workspace_bytes(b, s, h, d, n_cand)) if use_workspace else 0
    if ws_bytes < 0:
        _check("dsa_indexer_workspace_bytes", ws_bytes)
    if ws_bytes > 0:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        rc = lib.dsa_indexer_score_topk_ws(
            q.data_ptr(), kv_cache.data_ptr(), kv_cache.stride(0), wl.data_ptr(), float(w_scale),
            fr.data_ptr() if fr is not None else None, int(rope_mode), out.data_ptr(),
            b, s, h, d, rope_head_dim, n_cand, k_out, ratio, 1 if causal else 0, int(offset),
            ws.data_ptr(), ws_bytes, _stream(q))
        _check("dsa_indexer_score_topk_ws", rc)
        return out
    rc = lib.dsa_indexer_score_topk(
        q.data_ptr(), kv_cache.data_ptr(), kv_cache.stride(0), wl.data_ptr(), float(w_scale),
        fr.data_ptr() if fr is not None else None, int(rope_mode), out.data_ptr(),
        b, s, h, d, rope_head_dim, n_cand, k_out, ratio, 1 if causal else 0, int(offset),
        _stream(q))
    _check("dsa_indexer_score_topk", rc)
    return out


def indexer_scores(q: torch.Tensor, kv_cache: torch.Tensor, wl: torch.Tensor, w_scale: float,
                   freqs_cis: Optional[torch.Tensor], rope_head_dim: int, n_cand: int, ratio: int,
                   causal: bool, rope_mode: int = DSA_ROPE_TORCH_ROCM) -> torch.Tensor:
    """Task2 score stage: bf16 [b, s, n_cand] index scores (masked entries -inf when causal)."""
    lib = load()
    b, s, h, d = q.shape
    if kv_cache.stride(2) != 1 or kv_cache.stride(1) != d:
        kv_cache = kv_cache[:b, :n_cand].contiguous()
    q = q.contiguous()
    wl = wl.contiguous()
    fr = _freqs_view(freqs_cis, s, rope_head_dim) if freqs_cis is not None else None
    _require_gpu(q, kv_cache, wl, *([fr] if fr is not None else []))
    out = torch.empty(b, s, n_cand, dtype=torch.bfloat16, device=q.device)
    rc = lib.dsa_indexer_scores(
        q.data_ptr(), kv_cache.data_ptr(), kv_cache.stride(0), wl.data_ptr(), float(w_scale),
        fr.data_ptr() if fr is not None else None, int(rope_mode), out.data_ptr(),
        b, s, h, d, rope_head_dim, n_cand, ratio, 1 if causal else 0, _stream(q))
    _check("dsa_indexer_scores", rc)
    return out


def indexer_q_proj(qr: torch.Tensor, weight: torch.Tensor, freqs_cis: Optional[torch.Tensor],
                   head_dim: int, rope_head_dim: int,
                   rope_mode: int = DSA_ROPE_TORCH_ROCM) -> torch.Tensor:
    """q = qr . weight^T as bf16 [b, s, n/head_dim, head_dim] (F.linear's rounding), with
    RoPE on the last rope_head_dim channels of every head when freqs_cis (rows for the s
    positions) is given. qr: bf16 [b, s, k]; weight: bf16 [n, k]."""
    lib = load()
    if qr.dim() != 3 or weight.dim() != 2 or qr.shape[2] != weight.shape[1]:
        raise ValueError(f"qr {tuple(qr.shape)} and weight {tuple(weight.shape)} do not match")
    if qr.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("qr and weight must be bfloat16")
    b, s, k = qr.shape
    n = weight.shape[0]
    qr = qr.contiguous()
    weight = weight.contiguous()
    fr = _freqs_view(freqs_cis, s, rope_head_dim) if freqs_cis is not None else None
    _require_gpu(qr, weight, *([fr] if fr is not None else []))
    out = torch.empty(b, s, n // head_dim, head_dim, dtype=torch.bfloat16, device=qr.device)
    rc = lib.dsa_indexer_q_proj(qr.data_ptr(), weight.data_ptr(), fr.data_ptr() if fr is not None else None,
                                int(rope_mode), out.data_ptr(), b * s, n, k, head_dim, rope_head_dim,
                                max(s, 1), _stream(qr))
    _check("dsa_indexer_q_proj", rc)
    return out
