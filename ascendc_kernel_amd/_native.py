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

ABI_VERSION = 4

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
    "dsa_indexer_pack_projection_weights",
    "dsa_indexer_projections",
    "dsa_indexer_decode_projections",
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
    lib.dsa_indexer_pack_projection_weights.restype = ctypes.c_int
    lib.dsa_indexer_pack_projection_weights.argtypes = [
        _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp]
    lib.dsa_indexer_projections.restype = ctypes.c_int
    lib.dsa_indexer_projections.argtypes = [
        _c_vp, _c_vp, _c_vp, ctypes.c_int32, _c_vp, _c_vp, _c_vp, _c_vp,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]
    lib.dsa_indexer_decode_projections.restype = ctypes.c_int
    lib.dsa_indexer_decode_projections.argtypes = [
        _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]
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


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)

#: device type whose calls the modules serve from a cached launch plan (tests of the plan
#: logic on the CPU switch it)
PLAN_DEVICE_TYPE = "cuda"


def stream_handle(dev: torch.device) -> int:
    """hipStream_t of the current stream on `dev` as an int (the cheap query when torch has it)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


class Launch:
    """One prepared C-ABI call: the resolved entry point and its marshalled arguments, with
    the slots that change per call (fresh outputs) patched by index. Built on the first call
    with a given set of pointers and shapes; later calls skip the checks and the marshalling."""
    __slots__ = ("name", "fn", "args")

    def __init__(self, name: str, args: list):
        self.name = name
        lib = load()
        # The arguments are converted to ctypes objects once, by the entry point's declared
        # types; each call passes them to an untyped handle of the same symbol, which skips the
        # per-call conversion (about a third of a 14-argument call's cost).
        types = getattr(lib, name).argtypes
        if len(types) != len(args):
            raise TypeError(f"{name}: {len(args)} arguments for {len(types)} parameters")
        self.fn = lib[name]
        self.fn.restype = ctypes.c_int
        self.args = [t(a) for t, a in zip(types, args)]

    def set(self, slot: int, ptr: int) -> None:
        """Patch a pointer argument (a fresh output)."""
        self.args[slot].value = ptr

    def __call__(self) -> None:
        rc = self.fn(*self.args)
        if rc != 0:
            _check(self.name, rc)


def _require_gpu(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError("DSA kernels run on a HIP device only; got a tensor on "
                               f"{t.device}")
        if t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


class Prepared:
    """A checked, marshalled call and what it needs kept alive (inputs made contiguous,
    workspaces, the fp32 sink copy). run() allocates the fresh output, patches its pointer
    into the argument slot `out_slot` and launches."""
    __slots__ = ("launch", "out_slot", "out_shape", "out_dtype", "device", "keep", "_like", "_proto")

    def __init__(self, launch: Launch, out_slot: int, out_shape, out_dtype, device, keep):
        self.launch = launch
        self.out_slot = out_slot
        self.out_shape = tuple(out_shape)
        self.out_dtype = out_dtype
        self.device = device
        self.keep = keep
        # The output is allocated from the first kept input (a device tensor): empty_like when
        # it has the output's shape and dtype, else new_empty; both parse fewer arguments than
        # torch.empty(..., device=...), a measurable part of a steady-state call.
        proto = keep[0] if keep and isinstance(keep[0], torch.Tensor) and keep[0].device == device else None
        self._like = proto if (proto is not None and tuple(proto.shape) == self.out_shape
                               and proto.dtype == out_dtype and proto.is_contiguous()) else None
        self._proto = proto

    def run(self) -> torch.Tensor:
        if self._like is not None:
            out = torch.empty_like(self._like)
        elif self._proto is not None:
            out = self._proto.new_empty(self.out_shape, dtype=self.out_dtype)
        else:
            out = torch.empty(self.out_shape, dtype=self.out_dtype, device=self.device)
        launch = self.launch
        launch.args[self.out_slot].value = out.data_ptr()
        rc = launch.fn(*launch.args)
        if rc != 0:
            _check(launch.name, rc)
        return out


def prepare_sparse_attn(q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor,
                        attn_sink: torch.Tensor, softmax_scale: float,
                        variant: int = DSA_SA_AUTO) -> Prepared:
    """Checks and marshals dsa_sparse_attn_fwd[_i64] (output slot 4)."""
    load()
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
    args = [q.data_ptr(), kv.data_ptr(), idx.data_ptr(), sink.data_ptr(), None,
            b, m, h, d, kv.shape[1], idx.shape[2], float(softmax_scale), int(variant), stream_handle(dev)]
    return Prepared(Launch(fn, args), 4, (b, m, h, d), torch.bfloat16, dev, (q, kv, idx, sink))


def sparse_attn_fwd(q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor,
                    attn_sink: torch.Tensor, softmax_scale: float,
                    variant: int = DSA_SA_AUTO) -> torch.Tensor:
    """Task1 forward on the GPU; shapes as in reference/task1_v0_ref.py:5-24."""
    return prepare_sparse_attn(q, kv, topk_idxs, attn_sink, softmax_scale, variant).run()


def prepare_sparse_mla(q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor,
                       attn_sink: torch.Tensor, softmax_scale: float, v_dim: int,
                       split: bool = True) -> Prepared:
    """Checks and marshals dsa_sparse_mla_fwd[_i64][_ws] (output slot 4); the workspace of
    a split launch is allocated here and reused by every run() (calls on one stream)."""
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
    args = [q.data_ptr(), kv.data_ptr(), idx.data_ptr(), sink.data_ptr(), None,
            b, m, h, dqk, v_dim, kv.shape[2], kv.shape[1], idx.shape[2], float(softmax_scale)]
    # Few tokens (decode): the slot lists are split over workgroups whose partial
    # results go to a workspace from torch's caching allocator.
    ws_bytes = int(lib.dsa_sparse_mla_workspace_bytes(b, m, h, idx.shape[2])) if split else 0
    if ws_bytes < 0:
        _check("dsa_sparse_mla_workspace_bytes", ws_bytes)
    keep = [q, kv, idx, sink]
    if ws_bytes > 0:
        fn = "dsa_sparse_mla_fwd_i64_ws" if idx.dtype == torch.int64 else "dsa_sparse_mla_fwd_ws"
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        keep.append(ws)
        args += [ws.data_ptr(), ws_bytes]
    else:
        fn = "dsa_sparse_mla_fwd_i64" if idx.dtype == torch.int64 else "dsa_sparse_mla_fwd"
    args.append(stream_handle(dev))
    return Prepared(Launch(fn, args), 4, (b, m, h, v_dim), torch.bfloat16, dev, tuple(keep))


def sparse_mla_fwd(q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor,
                   attn_sink: torch.Tensor, softmax_scale: float, v_dim: int,
                   split: bool = True) -> torch.Tensor:
    """Sparse MLA on the GPU: q [b,m,h,d_qk], kv [b,n_kv,>=d_qk]; keys are kv[..., :d_qk],
    values kv[..., :v_dim]; returns bf16 [b,m,h,v_dim]. split=False keeps the one-pass
    kernel also where the library would split the slot lists (few tokens)."""
    return prepare_sparse_mla(q, kv, topk_idxs, attn_sink, softmax_scale, v_dim, split).run()


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


#: argument slots of dsa_indexer_score_topk[_ws] that change per call
SCORE_SLOT_Q, SCORE_SLOT_WL, SCORE_SLOT_OUT = 0, 3, 7


def prepare_indexer_score_topk(q: torch.Tensor, kv_cache: torch.Tensor, wl: torch.Tensor,
                               w_scale: float, freqs_cis: Optional[torch.Tensor], rope_head_dim: int,
                               n_cand: int, k_out: int, ratio: int, causal: bool, offset: int,
                               rope_mode: int = DSA_ROPE_TORCH_ROCM,
                               use_workspace: bool = True) -> Prepared:
    """Checks and marshals dsa_indexer_score_topk[_ws]: q, wl and out in the argument slots
    SCORE_SLOT_*; a workspace is allocated here and reused by every run()."""
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
    dev = _require_gpu(q, kv_cache, wl, *([fr] if fr is not None else []))
    args = [q.data_ptr(), kv_cache.data_ptr(), kv_cache.stride(0), wl.data_ptr(), float(w_scale),
            fr.data_ptr() if fr is not None else None, int(rope_mode), None,
            b, s, h, d, rope_head_dim, n_cand, k_out, ratio, 1 if causal else 0, int(offset)]
    ws_bytes = int(lib.dsa_indexer_workspace_bytes(b, s, h, d, n_cand)) if use_workspace else 0
    if ws_bytes < 0:
        _check("dsa_indexer_workspace_bytes", ws_bytes)
    keep = [q, kv_cache, wl, fr]
    if ws_bytes > 0:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        keep.append(ws)
        fn = "dsa_indexer_score_topk_ws"
        args += [ws.data_ptr(), ws_bytes]
    else:
        fn = "dsa_indexer_score_topk"
    args.append(stream_handle(dev))
    return Prepared(Launch(fn, args), SCORE_SLOT_OUT, (b, s, k_out), torch.int64, dev, tuple(keep))


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
    return prepare_indexer_score_topk(q, kv_cache, wl, w_scale, freqs_cis, rope_head_dim, n_cand, k_out,
                                      ratio, causal, offset, rope_mode, use_workspace).run()


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


def prepare_indexer_q_proj(qr: torch.Tensor, weight: torch.Tensor, freqs_cis: Optional[torch.Tensor],
                           head_dim: int, rope_head_dim: int,
                           rope_mode: int = DSA_ROPE_TORCH_ROCM) -> Prepared:
    """Checks and marshals dsa_indexer_q_proj (output q in slot 4)."""
    load()
    if qr.dim() != 3 or weight.dim() != 2 or qr.shape[2] != weight.shape[1]:
        raise ValueError(f"qr {tuple(qr.shape)} and weight {tuple(weight.shape)} do not match")
    if qr.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("qr and weight must be bfloat16")
    b, s, k = qr.shape
    n = weight.shape[0]
    qr = qr.contiguous()
    weight = weight.detach().contiguous()
    fr = _freqs_view(freqs_cis, s, rope_head_dim) if freqs_cis is not None else None
    dev = _require_gpu(qr, weight, *([fr] if fr is not None else []))
    args = [qr.data_ptr(), weight.data_ptr(), fr.data_ptr() if fr is not None else None, int(rope_mode), None,
            b * s, n, k, head_dim, rope_head_dim, max(s, 1), stream_handle(dev)]
    return Prepared(Launch("dsa_indexer_q_proj", args), 4, (b, s, n // head_dim, head_dim), torch.bfloat16,
                    dev, (qr, weight, fr))


def indexer_q_proj(qr: torch.Tensor, weight: torch.Tensor, freqs_cis: Optional[torch.Tensor],
                   head_dim: int, rope_head_dim: int,
                   rope_mode: int = DSA_ROPE_TORCH_ROCM) -> torch.Tensor:
    """q = qr . weight^T as bf16 [b, s, n/head_dim, head_dim] (F.linear's rounding), with
    RoPE on the last rope_head_dim channels of every head when freqs_cis (rows for the s
    positions) is given. qr: bf16 [b, s, k]; weight: bf16 [n, k]."""
    return prepare_indexer_q_proj(qr, weight, freqs_cis, head_dim, rope_head_dim, rope_mode).run()


def pack_projection_weights(wq: Optional[torch.Tensor], wproj: Optional[torch.Tensor]):
    """Fragment-packed copies of the indexer's projection weights for
    ``indexer_projections``: wq bf16 [n, 256] and wproj bf16 [n_w, dim] (either may be
    None). A permutation of the same bytes; pack once per weight version."""
    lib = load()
    ts = [t for t in (wq, wproj) if t is not None]
    if not ts:
        return None, None
    dev = _require_gpu(*ts)
    for t in ts:
        if t.dim() != 2 or t.dtype != torch.bfloat16:
            raise TypeError("projection weights must be 2-D bfloat16 tensors")
    wq_c = wq.detach().contiguous() if wq is not None else None
    wp_c = wproj.detach().contiguous() if wproj is not None else None
    wq_p = torch.empty_like(wq_c) if wq_c is not None else None
    wp_p = torch.empty_like(wp_c) if wp_c is not None else None
    rc = lib.dsa_indexer_pack_projection_weights(
        wq_c.data_ptr() if wq_c is not None else None,
        wq_c.shape[0] if wq_c is not None else 0, wq_c.shape[1] if wq_c is not None else 0,
        wp_c.data_ptr() if wp_c is not None else None,
        wp_c.shape[0] if wp_c is not None else 0, wp_c.shape[1] if wp_c is not None else 0,
        wq_p.data_ptr() if wq_p is not None else None, wp_p.data_ptr() if wp_p is not None else None,
        stream_handle(dev))
    _check("dsa_indexer_pack_projection_weights", rc)
    return wq_p, wp_p


#: argument slots of dsa_indexer_projections holding the outputs q and wl
PROJ_SLOT_Q, PROJ_SLOT_WL = 4, 7


def prepare_indexer_projections(qr: torch.Tensor, wq_packed: torch.Tensor, freqs_cis: Optional[torch.Tensor],
                                x: torch.Tensor, wproj_packed: torch.Tensor, head_dim: int, rope_head_dim: int,
                                rope_mode: int = DSA_ROPE_TORCH_ROCM):
    """Checks and marshals dsa_indexer_projections; returns (Launch, q_shape, wl_shape, keep)
    with the outputs in the argument slots PROJ_SLOT_Q and PROJ_SLOT_WL."""
    load()
    if qr.dim() != 3 or x.dim() != 3 or qr.shape[:2] != x.shape[:2]:
        raise ValueError(f"qr {tuple(qr.shape)} and x {tuple(x.shape)} do not match")
    if qr.dtype != torch.bfloat16 or x.dtype != torch.bfloat16:
        raise TypeError("qr and x must be bfloat16")
    b, s, k = qr.shape
    dim = x.shape[2]
    n = wq_packed.shape[0]
    n_w = wproj_packed.shape[0]
    if wq_packed.shape[1] != k or wproj_packed.shape[1] != dim:
        raise ValueError("packed weights do not match qr / x")
    qr = qr.contiguous()
    x = x.contiguous()
    fr = _freqs_view(freqs_cis, s, rope_head_dim) if freqs_cis is not None else None
    dev = _require_gpu(qr, x, wq_packed, wproj_packed, *([fr] if fr is not None else []))
    args = [qr.data_ptr(), wq_packed.data_ptr(), fr.data_ptr() if fr is not None else None, int(rope_mode),
            None, x.data_ptr(), wproj_packed.data_ptr(), None,
            b * s, n, k, dim, n_w, head_dim, rope_head_dim, max(s, 1), stream_handle(dev)]
    return (Launch("dsa_indexer_projections", args), (b, s, n // head_dim, head_dim), (b, s, n_w),
            (qr, x, wq_packed, wproj_packed, fr))


def indexer_projections(qr: torch.Tensor, wq_packed: torch.Tensor, freqs_cis: Optional[torch.Tensor],
                        x: torch.Tensor, wproj_packed: torch.Tensor, head_dim: int, rope_head_dim: int,
                        rope_mode: int = DSA_ROPE_TORCH_ROCM):
    """Both indexer projections in one launch: q = RoPE(qr . wq^T) as bf16
    [b, s, n/head_dim, head_dim] and wl = x . wproj^T as bf16 [b, s, n_w], from the
    packed weights of ``pack_projection_weights``. qr: bf16 [b, s, 256]; x: bf16 [b, s, dim]."""
    launch, q_shape, wl_shape, _keep = prepare_indexer_projections(qr, wq_packed, freqs_cis, x, wproj_packed,
                                                                   head_dim, rope_head_dim, rope_mode)
    q = torch.empty(q_shape, dtype=torch.bfloat16, device=qr.device)
    wl = torch.empty(wl_shape, dtype=torch.bfloat16, device=qr.device)
    launch.set(PROJ_SLOT_Q, q.data_ptr())
    launch.set(PROJ_SLOT_WL, wl.data_ptr())
    launch()
    return q, wl


#: argument slots of the two outputs of dsa_indexer_decode_projections
DECODE_SLOT_Q = 4
DECODE_SLOT_WL = 5


def prepare_indexer_decode_projections(qr: torch.Tensor, wq: torch.Tensor, x: torch.Tensor, wproj: torch.Tensor):
    """Checks and marshals dsa_indexer_decode_projections; returns (Launch, q_shape,
    wl_shape, keep) with the outputs in the argument slots DECODE_SLOT_Q / DECODE_SLOT_WL.
    qr: bf16 [b, s, 1536], x: bf16 [b, s, 7168] with b * s <= 16; wq [n_q, 1536] and
    wproj [n_w, 7168] the Linear weights as they are."""
    load()
    if qr.dim() != 3 or x.dim() != 3 or qr.shape[:2] != x.shape[:2]:
        raise ValueError(f"qr {tuple(qr.shape)} and x {tuple(x.shape)} do not match")
    if wq.dim() != 2 or wproj.dim() != 2 or wq.shape[1] != qr.shape[2] or wproj.shape[1] != x.shape[2]:
        raise ValueError(f"weights {tuple(wq.shape)} / {tuple(wproj.shape)} do not match qr / x")
    for t in (qr, x, wq, wproj):
        if t.dtype != torch.bfloat16:
            raise TypeError("qr, x and both weights must be bfloat16")
    b, s, k_q = qr.shape
    k_w = x.shape[2]
    qr, x, wq, wproj = qr.contiguous(), x.contiguous(), wq.contiguous(), wproj.contiguous()
    dev = _require_gpu(qr, x, wq, wproj)
    args = [qr.data_ptr(), wq.data_ptr(), x.data_ptr(), wproj.data_ptr(), None, None,
            b * s, wq.shape[0], k_q, wproj.shape[0], k_w, stream_handle(dev)]
    return (Launch("dsa_indexer_decode_projections", args), (b, s, wq.shape[0]), (b, s, wproj.shape[0]),
            (qr, x, wq, wproj))


def indexer_decode_projections(qr: torch.Tensor, wq: torch.Tensor, x: torch.Tensor, wproj: torch.Tensor):
    """q = qr . wq^T as bf16 [b, s, n_q] and wl = x . wproj^T as bf16 [b, s, n_w] for
    b * s <= 16 tokens, in hipBLASLt's local-split rounding (no RoPE)."""
    launch, q_shape, wl_shape, _keep = prepare_indexer_decode_projections(qr, wq, x, wproj)
    q = torch.empty(q_shape, dtype=torch.bfloat16, device=qr.device)
    wl = torch.empty(wl_shape, dtype=torch.bfloat16, device=qr.device)
    launch.set(DECODE_SLOT_Q, q.data_ptr())
    launch.set(DECODE_SLOT_WL, wl.data_ptr())
    launch()
    return q, wl
