"""qsa_sparse_attention_noalloc (split partials in the library's per-GPU
scratch) against qsa_sparse_attention (partials in a caller workspace),
through the C ABI: identical bits, on two calls in a row, the second with a
smaller input, both with split partials in use. Sizes beyond the scratch fail
with QSA_ERR_WORKSPACE before anything is launched."""

import ctypes

import pytest
import torch

from qsa_vllm_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(seed, rows, hq, hkv, dim, width, blocks=96, page=16):
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(blocks, page, hkv, 2 * dim, generator=g).to(torch.bfloat16).to(DEV)
    idx = torch.randint(0, blocks * page, (rows, width), generator=g, dtype=torch.int32)
    counts = torch.randint(0, width + 1, (rows,), generator=g, dtype=torch.int32)
    counts[0] = width
    for r in range(rows):
        idx[r, int(counts[r]):] = -1
    return dict(q=torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16).to(DEV),
                k=kv[..., :dim], v=kv[..., dim:], idx=idx.to(DEV), counts=counts.to(DEV),
                gate=torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16).to(DEV),
                t2r=torch.zeros(rows, dtype=torch.int32, device=DEV),
                table=torch.zeros(1, 1, dtype=torch.int32, device=DEV))


def _args(c, out, splits):
    q, k, v, idx, gate = c["q"], c["k"], c["v"], c["idx"], c["gate"]
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    return [p(q), q.stride(0), q.stride(1), q.shape[0], q.shape[1], q.shape[2],
            p(k), k.stride(0), k.stride(1), k.stride(2),
            p(v), v.stride(0), v.stride(1), v.stride(2),
            k.shape[0], k.shape[1], k.shape[2],
            p(idx), idx.stride(0), idx.shape[1],
            p(c["table"]), c["table"].stride(0), 1, 1,
            p(c["t2r"]), p(c["counts"]),
            p(out), out.stride(0), out.stride(1),
            p(gate), gate.stride(0), gate.stride(1), gate.stride(2),
            1, splits]


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _with_workspace(c, splits):
    lib = _lib.load()
    out = torch.full_like(c["q"], float("nan"))
    rows, hq, dim = c["q"].shape
    nbytes = lib.qsa_sparse_attention_workspace_bytes(rows, hq, dim, splits)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    _lib.check(lib.qsa_sparse_attention(*_args(c, out, splits), ctypes.c_void_p(ws.data_ptr()),
                                        nbytes, _stream()), "qsa_sparse_attention")
    return out


def _no_alloc(c, splits):
    out = torch.full_like(c["q"], float("nan"))
    _lib.check(_lib.load().qsa_sparse_attention_noalloc(*_args(c, out, splits), _stream()),
               "qsa_sparse_attention_noalloc")
    return out


def test_noalloc_matches_workspace_entry_point():
    lib = _lib.load()
    big = _case(1, rows=96, hq=16, hkv=2, dim=128, width=600)
    small = _case(2, rows=20, hq=16, hkv=2, dim=64, width=300)
    for what, c, splits in (("first call", big, 4), ("second, smaller call", small, 2)):
        rows, hq, dim = c["q"].shape
        assert 0 < lib.qsa_sparse_attention_workspace_bytes(rows, hq, dim, splits) \
            <= _lib.SPARSE_ATTENTION_SCRATCH_BYTES
        print(f"[case] noalloc {what}: rows={rows} hq={hq} dim={dim} splits={splits}", flush=True)
        got = _no_alloc(c, splits)
        want = _with_workspace(c, splits)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all(), what
        assert torch.equal(got, want), what


def test_noalloc_rejects_partials_beyond_scratch():
    lib = _lib.load()
    c = _case(3, rows=64, hq=16, hkv=2, dim=128, width=64)
    splits = 128   # 128 * 64 * 16 * (128 + 1) * 4 bytes > 32 MiB
    assert lib.qsa_sparse_attention_workspace_bytes(64, 16, 128, splits) > \
        _lib.SPARSE_ATTENTION_SCRATCH_BYTES
    out = torch.full_like(c["q"], float("nan"))
    status = lib.qsa_sparse_attention_noalloc(*_args(c, out, splits), _stream())
    torch.cuda.synchronize()
    assert status == _lib.QSA_ERR_WORKSPACE
    assert b"scratch" in lib.qsa_last_error()
    assert torch.isnan(out.float()).all(), "nothing may be launched"
