"""The C-ABI library: loads, exports what include/dsa_abi.h declares, and rejects
bad arguments on the host (these calls return before any HIP call)."""
import ctypes
import os
import re

import pytest

from conftest import REPO
from ascendc_kernel_amd import _native


def _declared():
    text = open(os.path.join(REPO, "include", "dsa_abi.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(dsa_\w+)\s*\(", text, re.M)))


def test_library_present_and_loads():
    lib = _native.load()
    assert lib.dsa_abi_version() == _native.ABI_VERSION


def test_exports_every_declared_symbol():
    decl = _declared()
    assert set(decl) == set(_native.EXPORTS)
    lib = ctypes.CDLL(_native.lib_path())
    for name in decl:
        assert hasattr(lib, name), name


def test_strerror():
    lib = _native.load()
    assert lib.dsa_strerror(0) == b"ok"
    for code in (-1, -2, -3, -4, -5, -6, -7):
        assert lib.dsa_strerror(code) not in (b"ok", b"unknown error")
    assert lib.dsa_strerror(-99) == b"unknown error"


def _sa(lib, **kw):
    a = dict(q=16, kv=16, idx=16, sink=16, out=16, b=1, m=1, h=64, d=128, n_kv=32, topk=16,
             scale=0.1, variant=0)
    a.update(kw)
    return lib.dsa_sparse_attn_fwd(a["q"], a["kv"], a["idx"], a["sink"], a["out"], a["b"], a["m"],
                                   a["h"], a["d"], a["n_kv"], a["topk"], a["scale"], a["variant"], None)


def test_sparse_attn_host_checks():
    lib = _native.load()
    assert _sa(lib, b=-1) == -2
    assert _sa(lib, topk=0) == -2
    assert _sa(lib, n_kv=0) == -2
    assert _sa(lib, d=64) == -3
    assert _sa(lib, h=24) == -3
    assert _sa(lib, variant=1, n_kv=33) == -3
    assert _sa(lib, variant=7) == -3
    assert _sa(lib, b=0) == 0 and _sa(lib, m=0) == 0
    assert _sa(lib, q=None) == -1
    assert _sa(lib, out=None) == -1
    assert _sa(lib, q=8) == -6


def _ix(lib, **kw):
    a = dict(q=16, kv=16, kvbs=650 * 64, wl=16, scale=0.03, fr=16, mode=1, out=16, b=1, s=8,
             h=16, d=64, rd=32, T=650, K=128, ratio=4, causal=1, offset=0)
    a.update(kw)
    return lib.dsa_indexer_score_topk(a["q"], a["kv"], a["kvbs"], a["wl"], a["scale"], a["fr"],
                                      a["mode"], a["out"], a["b"], a["s"], a["h"], a["d"], a["rd"],
                                      a["T"], a["K"], a["ratio"], a["causal"], a["offset"], None)


def test_indexer_host_checks():
    lib = _native.load()
    assert _ix(lib, K=700) == -2
    assert _ix(lib, T=0) == -2
    assert _ix(lib, ratio=0) == -2
    assert _ix(lib, h=64) == -3
    assert _ix(lib, d=128) == -3
    assert _ix(lib, K=512) == -3
    assert _ix(lib, mode=5) == -3
    assert _ix(lib, rd=33) == -2
    assert _ix(lib, kvbs=100) == -2
    assert _ix(lib, s=0) == 0
    assert _ix(lib, q=None) == -1
    assert _ix(lib, wl=24) == -6


def test_rope_host_checks():
    lib = _native.load()
    assert lib.dsa_indexer_rope(16, 16, 1, 4, 16, 64, 33, 1, None) == -2
    assert lib.dsa_indexer_rope(16, 16, 1, 4, 16, 64, 80, 1, None) == -2
    assert lib.dsa_indexer_rope(16, 16, 1, 4, 16, 64, 32, 3, None) == -3
    assert lib.dsa_indexer_rope(16, 16, 0, 4, 16, 64, 32, 1, None) == 0
    assert lib.dsa_indexer_rope(None, 16, 1, 4, 16, 64, 32, 1, None) == -1


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setenv("DSA_MI355X_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="missing"):
        _native.load()


def _mla(lib, **kw):
    a = dict(q=16, kv=16, idx=16, sink=16, out=16, b=1, m=4, h=128, dqk=576, dv=512, kv_dim=576,
             n_kv=100, topk=64, scale=576 ** -0.5)
    a.update(kw)
    return lib.dsa_sparse_mla_fwd(a["q"], a["kv"], a["idx"], a["sink"], a["out"], a["b"], a["m"], a["h"],
                                  a["dqk"], a["dv"], a["kv_dim"], a["n_kv"], a["topk"], a["scale"], None)


def test_sparse_mla_host_checks():
    """Every rejection happens before any HIP call, so it runs without a GPU."""
    lib = _native.load()
    assert _mla(lib, b=-1) == -2
    assert _mla(lib, n_kv=0) == -2
    assert _mla(lib, topk=0) == -2
    assert _mla(lib, dqk=512) == -3          # only d_qk 576 / d_v 512 are built
    assert _mla(lib, dv=576) == -3
    assert _mla(lib, kv_dim=512) == -3       # rows narrower than the keys
    assert _mla(lib, kv_dim=580) == -3       # row stride must be a multiple of 8 channels
    assert _mla(lib, h=48) == -3             # 64..128 heads in steps of 16
    assert _mla(lib, h=144) == -3
    assert _mla(lib, h=72) == -3
    assert _mla(lib, topk=2049) == -3
    assert _mla(lib, scale=0.0) == -3
    assert _mla(lib, scale=float("inf")) == -3
    assert _mla(lib, n_kv=(1 << 21) + 1) == -3
    assert _mla(lib, b=0) == 0 and _mla(lib, m=0) == 0
    assert _mla(lib, q=None) == -1
    assert _mla(lib, out=None) == -1
    assert _mla(lib, kv=24) == -6


def test_int64_index_entry_points_host_checks():
    """dsa_sparse_attn_fwd_i64 / dsa_sparse_mla_fwd_i64 share the int32 entry points'
    checks (they differ only in how the kernels read topk_idxs)."""
    lib = _native.load()
    a = [16, 16, 16, 16, 16, 1, 1, 64, 128, 32, 16, 0.1, 0, None]
    f = lib.dsa_sparse_attn_fwd_i64
    assert f(*a[:5], -1, *a[6:]) == -2                   # b < 0
    assert f(*a[:8], 64, *a[9:]) == -3                   # d != 128
    assert f(*a[:12], 7, None) == -3                     # unknown variant
    assert f(*a[:9], 33, *a[10:12], 1, None) == -3       # multiplicity variant needs n_kv <= 32
    assert f(*a[:5], 0, *a[6:]) == 0                     # empty batch: nothing to do
    assert f(None, *a[1:]) == -1
    assert f(8, *a[1:]) == -6
    m = [16, 16, 16, 16, 16, 1, 1, 128, 576, 512, 576, 100, 64, 576 ** -0.5, None]
    g = lib.dsa_sparse_mla_fwd_i64
    assert g(*m[:5], -1, *m[6:]) == -2
    assert g(*m[:8], 512, *m[9:]) == -3                  # d_qk != 576
    assert g(*m[:12], 2049, *m[13:]) == -3               # topk > 2048
    assert g(*m[:6], 0, *m[7:]) == 0
    assert g(*m[:2], None, *m[3:]) == -1                 # no topk_idxs
    assert g(*m[:4], None, *m[5:]) == -1                 # no out
    # a batch's kv rows beyond 4 GiB: 32-bit row offsets would wrap
    assert g(*m[:10], 1024, 1 << 21, *m[12:]) == -3


def test_sparse_mla_workspace_entry_points_host_checks():
    """dsa_sparse_mla_fwd_ws / _i64_ws check shapes like dsa_sparse_mla_fwd and reject a
    negative workspace size; the workspace query is 0 for empty requests and a negative
    DSA_ERR_* code (never a size) for invalid ones."""
    lib = _native.load()
    m = [16, 16, 16, 16, 16, 1, 1, 128, 576, 512, 576, 100, 64, 576 ** -0.5, 16, 1 << 20, None]
    for f in (lib.dsa_sparse_mla_fwd_ws, lib.dsa_sparse_mla_fwd_i64_ws):
        assert f(*m[:5], -1, *m[6:]) == -2
        assert f(*m[:8], 512, *m[9:]) == -3
        assert f(*m[:15], -1, None) == -2
        assert f(*m[:6], 0, *m[7:]) == 0
        assert f(*m[:2], None, *m[3:]) == -1
    assert lib.dsa_sparse_mla_workspace_bytes(0, 1, 128, 2048) == 0
    assert lib.dsa_sparse_mla_workspace_bytes(1, 1, 128, 0) == -2
    assert lib.dsa_sparse_mla_workspace_bytes(-1, 1, 128, 64) == -2


def _ixw(lib, **kw):
    a = dict(q=16, kv=16, kvbs=8192 * 128, wl=16, scale=0.011, fr=16, mode=1, out=16, b=1, s=8,
             h=64, d=128, rd=64, T=8192, K=2048, ratio=1, causal=1, offset=0, ws=16, wsb=1 << 20)
    a.update(kw)
    return lib.dsa_indexer_score_topk_ws(a["q"], a["kv"], a["kvbs"], a["wl"], a["scale"], a["fr"], a["mode"],
                                         a["out"], a["b"], a["s"], a["h"], a["d"], a["rd"], a["T"], a["K"],
                                         a["ratio"], a["causal"], a["offset"], a["ws"], a["wsb"], None)


def test_wide_indexer_host_checks():
    lib = _native.load()
    assert _ixw(lib, T=8196, kvbs=8196 * 128) == -3  # more than 8192 candidates
    assert _ixw(lib, T=8192, K=4096) == -3           # top-k beyond 2048
    assert _ixw(lib, K=8193) == -2                   # k > candidates
    assert _ixw(lib, kvbs=100) == -2
    assert _ixw(lib, rd=130) == -2
    assert _ixw(lib, wsb=-1) == -2
    assert _ixw(lib, ws=24) == -6                    # workspace must be 16-byte aligned
    assert _ixw(lib, out=None) == -1
    assert _ixw(lib, s=0) == 0


def test_workspace_bytes():
    lib = _native.load()
    assert lib.dsa_indexer_workspace_bytes(1, 8192, 64, 128, 8192) == 8192 * 8192 * 2
    assert lib.dsa_indexer_workspace_bytes(2, 100, 64, 128, 512) == 2 * 100 * 512 * 2
    assert lib.dsa_indexer_workspace_bytes(1, 3, 64, 128, 8190) == 3 * 8192 * 2   # rows padded to 4 keys
    assert lib.dsa_indexer_workspace_bytes(8, 2600, 16, 64, 650) == 0   # the 16-head kernel needs none
    assert lib.dsa_indexer_workspace_bytes(-1, 8, 64, 128, 64) == -2


def test_indexer_scores_host_checks():
    lib = _native.load()
    args = [16, 16, 650 * 64, 16, 0.03, 16, 1, 16, 1, 8, 16, 64, 32, 650, 4, 1, None]
    assert lib.dsa_indexer_scores(*args[:7], None, *args[8:]) == -1   # no score buffer
    bad = list(args)
    bad[7] = 17                                                          # odd address for bf16 scores
    assert lib.dsa_indexer_scores(*bad) == -6
    bad = list(args)
    bad[13] = 0                                                          # no candidates
    assert lib.dsa_indexer_scores(*bad) == -2


def test_indexer_noalloc_host_checks():
    """dsa_indexer_score_topk_noalloc: requests beyond the static scratch array are refused
    with DSA_ERR_SCRATCH before anything runs; shape and pointer checks as the _ws form."""
    lib = _native.load()

    def f(**kw):
        a = dict(q=16, kv=16, kvbs=8192 * 128, wl=16, scale=0.011, fr=16, mode=1, out=16, b=1, s=8192,
                 h=64, d=128, rd=64, T=8192, K=2048, ratio=1, causal=1, offset=0)
        a.update(kw)
        return lib.dsa_indexer_score_topk_noalloc(
            a["q"], a["kv"], a["kvbs"], a["wl"], a["scale"], a["fr"], a["mode"], a["out"], a["b"],
            a["s"], a["h"], a["d"], a["rd"], a["T"], a["K"], a["ratio"], a["causal"], a["offset"], None)

    assert f() == -7                      # 8192 x 8192 keys: 128 MiB > 16 MiB
    assert f(s=1025, T=8192) == -7        # one token row beyond 8,388,608 keys
    assert lib.dsa_strerror(-7) == b"request exceeds the library's static scratch buffer"
    assert f(b=-1) == -2
    assert f(out=None) == -1
    assert f(s=0) == 0


def test_q_proj_host_checks():
    lib = _native.load()

    def f(**kw):
        a = dict(qr=16, w=16, fr=16, mode=1, q=16, m=2600, n=1024, k=256, d=64, rd=32, s=2600)
        a.update(kw)
        return lib.dsa_indexer_q_proj(a["qr"], a["w"], a["fr"], a["mode"], a["q"], a["m"], a["n"], a["k"],
                                      a["d"], a["rd"], a["s"], None)

    assert f(m=-1) == -2
    assert f(k=250) == -3          # k % 32
    assert f(n=1000, d=40) == -3   # n % 256
    assert f(rd=30) == -3          # rotated channels not on an 8-channel boundary
    assert f(rd=66) == -2          # rd > head_dim
    assert f(m=2599) == -2         # m not a multiple of s_len
    assert f(mode=5) == -3
    assert f(m=0) == 0
    assert f(q=None) == -1
    assert f(fr=24) == -6          # table not 16-byte aligned


def _proj(lib, **kw):
    a = dict(qr=16, wq=16, fr=16, mode=1, q=16, x=16, wp=16, wl=16, m=64, n=1024, k=256, dim=1024, n_w=16,
             d=64, rd=32, s=64)
    a.update(kw)
    return lib.dsa_indexer_projections(a["qr"], a["wq"], a["fr"], a["mode"], a["q"], a["x"], a["wp"], a["wl"],
                                       a["m"], a["n"], a["k"], a["dim"], a["n_w"], a["d"], a["rd"], a["s"], None)


def test_projections_host_checks():
    lib = _native.load()
    assert _proj(lib, m=-1) == -2
    assert _proj(lib, n=1000) == -2                 # n % head_dim
    assert _proj(lib, m=65) == -2                   # m % s_len
    assert _proj(lib, k=512) == -3                  # k = 256 only
    assert _proj(lib, d=128, n=1024) == -3          # head_dim 64 only
    assert _proj(lib, dim=2048) == -3 and _proj(lib, n_w=32) == -3
    assert _proj(lib, rd=64) == -3 and _proj(lib, mode=5) == -3
    assert _proj(lib, rd=33) == -2
    assert _proj(lib, m=0) == 0
    for name in ("qr", "wq", "q", "x", "wp", "wl"):
        assert _proj(lib, **{name: None}) == -1, name
    assert _proj(lib, x=8) == -6 and _proj(lib, wl=4) == -6 and _proj(lib, fr=8) == -6
    assert _proj(lib, m=2 ** 21, s=2 ** 21) == -3   # 32-bit buffer offsets


def test_pack_projection_weights_host_checks():
    lib = _native.load()
    f = lib.dsa_indexer_pack_projection_weights
    assert f(None, 0, 0, None, 0, 0, None, None, None) == 0          # nothing to pack
    assert f(16, 1024, 256, None, 0, 0, None, None, None) == -1      # wq without its output
    assert f(16, 1024, 512, None, 0, 0, 16, None, None) == -3        # k = 256 only
    assert f(16, 1000, 256, None, 0, 0, 16, None, None) == -3        # n % 64
    assert f(16, -1, 256, None, 0, 0, 16, None, None) == -2
    assert f(None, 0, 0, 16, 20, 1024, None, 16, None) == -3         # n_w % 16
    assert f(None, 0, 0, 16, 16, 1000, None, 16, None) == -3         # dim % 32
    assert f(8, 1024, 256, None, 0, 0, 16, None, None) == -6


def _dproj(lib, m=1, n_q=8192, k_q=1536, n_w=64, k_w=7168, **ptrs):
    p = dict(qr=16, wq=16, x=16, wp=16, q=16, wl=16)
    p.update(ptrs)
    return lib.dsa_indexer_decode_projections(p["qr"], p["wq"], p["x"], p["wp"], p["q"], p["wl"],
                                              m, n_q, k_q, n_w, k_w, None)


def test_decode_projections_host_checks():
    """Shape, pointer and alignment errors of dsa_indexer_decode_projections come back before
    anything is launched (no GPU needed)."""
    lib = _native.load()
    assert _dproj(lib, m=-1) == -2 and _dproj(lib, n_q=0) == -2 and _dproj(lib, k_w=-5) == -2
    assert _dproj(lib, m=17) == -3                  # 1..16 tokens
    assert _dproj(lib, k_q=1024) == -3 and _dproj(lib, k_w=4096) == -3   # the measured depths only
    assert _dproj(lib, n_q=8160) == -3 and _dproj(lib, n_w=40) == -3     # 64-channel / 16-channel tiles
    assert _dproj(lib, m=0) == 0                    # nothing to do
    for name in ("qr", "wq", "x", "wp", "q", "wl"):
        assert _dproj(lib, **{name: None}) == -1, name
    assert _dproj(lib, qr=8) == -6 and _dproj(lib, wp=24) == -6 and _dproj(lib, q=17) == -6
