"""qsa_sparse_attention_noalloc (split partials in the library's per-GPU
scratch) against qsa_sparse_attention (partials in a caller workspace),
through the C ABI: identical bits, on two calls in a row, the second with a
smaller input, both with split partials in use, for physical and logical
indices. In a fresh process whose first noalloc call is made under HIP graph
capture, replays on new inputs give the workspace entry point's bits. Sizes
beyond the scratch fail with QSA_ERR_WORKSPACE before anything is launched."""

import ctypes
import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from qsa_vllm_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(seed, rows, hq, hkv, dim, width, blocks=96, page=16, physical=True):
    """Physical slots with valid counts, or logical token ids of three
    requests (8 pages each) with padding rows and no counts."""
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(blocks, page, hkv, 2 * dim, generator=g).to(torch.bfloat16).to(DEV)
    if physical:
        idx = torch.randint(0, blocks * page, (rows, width), generator=g, dtype=torch.int32)
        counts = torch.randint(0, width + 1, (rows,), generator=g, dtype=torch.int32)
        counts[0] = width
        for r in range(rows):
            idx[r, int(counts[r]):] = -1
        t2r = torch.zeros(rows, dtype=torch.int32)
        table = torch.zeros(1, 1, dtype=torch.int32)
    else:
        idx = torch.randint(-2, 8 * page + 4, (rows, width), generator=g, dtype=torch.int32)
        counts = None
        t2r = torch.randint(-1, 3, (rows,), generator=g, dtype=torch.int32)
        table = torch.randperm(blocks, generator=g)[:24].view(3, 8).to(torch.int32)
        table[1, 6:] = -1
    return dict(q=torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16).to(DEV),
                k=kv[..., :dim], v=kv[..., dim:], idx=idx.to(DEV),
                counts=None if counts is None else counts.to(DEV),
                gate=torch.randn(rows, hq, dim, generator=g).to(torch.bfloat16).to(DEV),
                t2r=t2r.to(DEV), table=table.to(DEV), physical=int(physical))


def _args(c, out, splits):
    q, k, v, idx, gate = c["q"], c["k"], c["v"], c["idx"], c["gate"]
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    return [p(q), q.stride(0), q.stride(1), q.shape[0], q.shape[1], q.shape[2],
            p(k), k.stride(0), k.stride(1), k.stride(2),
            p(v), v.stride(0), v.stride(1), v.stride(2),
            k.shape[0], k.shape[1], k.shape[2],
            p(idx), idx.stride(0), idx.shape[1],
            p(c["table"]), c["table"].stride(0), c["table"].shape[1], c["table"].shape[0],
            p(c["t2r"]), None if c["counts"] is None else p(c["counts"]),
            p(out), out.stride(0), out.stride(1),
            p(gate), gate.stride(0), gate.stride(1), gate.stride(2),
            c["physical"], splits]


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


@pytest.mark.parametrize("physical", [True, False])
def test_noalloc_matches_workspace_entry_point(physical):
    lib = _lib.load()
    big = _case(1, rows=96, hq=16, hkv=2, dim=128, width=600, physical=physical)
    small = _case(2, rows=20, hq=16, hkv=2, dim=64, width=300, physical=physical)
    for what, c, splits in (("first call", big, 4), ("second, smaller call", small, 2)):
        rows, hq, dim = c["q"].shape
        assert 0 < lib.qsa_sparse_attention_workspace_bytes(rows, hq, dim, splits) \
            <= _lib.SPARSE_ATTENTION_SCRATCH_BYTES
        print(f"[case] noalloc {what}: physical={physical} rows={rows} hq={hq} dim={dim} "
              f"splits={splits}", flush=True)
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


_CAPTURE_CHILD = """
import sys
import torch
sys.path.insert(0, {test_dir!r})
import test_zz_no_alloc as t
from qsa_vllm_amd import _lib

lib = _lib.load()
for physical in (True, False):
    c = t._case(5, rows=48, hq=16, hkv=2, dim=128, width=400, physical=physical)
    out = torch.full_like(c["q"], float("nan"))
    graph = torch.cuda.CUDAGraph()
    print(f"[child] capture of the first noalloc call, physical={{physical}}", flush=True)
    with torch.cuda.graph(graph):
        status = lib.qsa_sparse_attention_noalloc(*t._args(c, out, 4), t._stream())
    assert status == _lib.QSA_OK, lib.qsa_last_error()
    for seed in (6, 7):
        new = t._case(seed, rows=48, hq=16, hkv=2, dim=128, width=400, physical=physical)
        for name in ("q", "idx", "gate", "t2r"):
            c[name].copy_(new[name])
        if physical:
            c["counts"].copy_(new["counts"])
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = t._with_workspace(c, 4)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all(), (physical, seed)
        assert torch.equal(out, want), (physical, seed)
        print(f"[child] replay seed={{seed}} physical={{physical}} equal", flush=True)
print("child ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """The scratch address is looked up on a device's first noalloc call; here
    that call is made under HIP graph capture, in a fresh process, and the
    graph is replayed on new inputs."""
    test_dir = str(Path(__file__).resolve().parent)
    repo = str(Path(__file__).resolve().parent.parent)
    env = dict(os.environ, PYTHONPATH=repo + os.pathsep + os.environ.get("PYTHONPATH", ""))
    print("[case] noalloc first call under graph capture (child process)", flush=True)
    proc = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD.format(test_dir=test_dir)],
                          cwd=repo, env=env, capture_output=True, text=True, timeout=100)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0 and "child ok" in proc.stdout
