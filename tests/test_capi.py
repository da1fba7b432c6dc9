"""C-ABI library checks that need no GPU: exports, signatures, argument errors."""

import ctypes
import re
import subprocess
import shutil
from pathlib import Path

import pytest

from qsa_vllm_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qsa_hip.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qsa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.library_path()))
    names = header_functions()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    assert sorted(_lib.SIGNATURES) == header_functions()
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, argtypes) in _lib.SIGNATURES.items():
        decl = re.search(rf"\b{name}\s*\((.*?)\);", text, flags=re.S).group(1).strip()
        nargs = 0 if decl in ("", "void") else len(decl.split(","))
        assert nargs == len(argtypes), name


def test_abi_version_and_clean_error():
    lib = _lib.load()
    assert lib.qsa_abi_version() == _lib.ABI_VERSION
    assert lib.qsa_last_error() is not None


def _attn_args(**over):
    a = dict(q=1 << 20, qr=256, qh=128, rows=4, hq=16, d=128, k=1 << 21, kb=4096, kt=256, kh=128,
             v=(1 << 21) + 256, vb=4096, vt=256, vh=128, nblk=8, page=16, hkv=2, idx=1 << 22,
             idxr=64, width=64, table=1 << 23, tabr=4, tabw=4, nreq=4, t2r=1 << 24, counts=None,
             out=1 << 25, outr=2048, outh=128, gate=None, gr=0, gh=0, gd=0, phys=1, splits=1,
             ws=None, wsb=0, stream=None)
    a.update(over)
    return list(a.values())


def test_attention_argument_errors_need_no_launch():
    lib = _lib.load()
    f = lib.qsa_sparse_attention
    assert f(*_attn_args(rows=0)) == 0
    assert f(*_attn_args(d=96)) == -2
    assert b"head_dim" in lib.qsa_last_error()
    assert f(*_attn_args(hq=12, hkv=8)) == -2          # 12 % 8 != 0
    assert f(*_attn_args(hq=48, hkv=2)) == -2          # group 24 neither divides nor multiplies 16
    assert f(*_attn_args(splits=4)) == -4              # split partials need a workspace
    assert f(*_attn_args(q=(1 << 20) + 2)) == -1       # misaligned q
    assert f(*_attn_args(phys=0, table=None)) == -1


def test_topk_argument_errors_need_no_launch():
    lib = _lib.load()
    args = [1 << 20, 64, 0, 64, 1 << 21, 1 << 22, 64, 8, None, 0, None]
    assert lib.qsa_topk(*args) == 0                     # zero rows
    args[2] = 4
    args[7] = 0
    assert lib.qsa_topk(*args) == -1                    # topk must be positive
    assert lib.qsa_topk_workspace_bytes(4, 16384, 128) == 0
    assert lib.qsa_topk_workspace_bytes(4, 65536, 128) == 4 * 8 * 128 * 4
    args = [1 << 20, 70000, 4, 70000, 1 << 21, 1 << 22, 64, 128, None, 0, None]
    assert lib.qsa_topk(*args) == -4                    # long rows need the partition workspace


def test_gated_norm_hidden_sizes_checked_before_the_row_split():
    """One supported hidden set for both launch paths (a workgroup per token
    below 1024 rows, 16-token tiles above): 3072 is refused at any row count."""
    lib = _lib.load()
    p = [1 << 20, 4096, None, 0, None, 0, 1 << 21, 1 << 22, 1 << 23, 1 << 24, 1 << 25, 4096]
    for rows in (16, 4096):
        for hidden, want in ((3072, -2), (1536, -2), (8192, -2), (256, -2)):
            args = p + [rows, hidden, 16, 1e-6, None, 0, None]
            assert lib.qsa_gated_norm(*args) == want, (rows, hidden)
            assert b"hidden size" in lib.qsa_last_error()
    assert lib.qsa_gated_norm(*(p + [0, 3072, 16, 1e-6, None, 0, None])) == 0   # no rows


def test_workspace_and_split_helpers():
    lib = _lib.load()
    assert lib.qsa_sparse_attention_workspace_bytes(64, 16, 128, 1) == 0
    assert lib.qsa_sparse_attention_workspace_bytes(64, 16, 128, 4) == 4 * 64 * 16 * (128 + 1) * 4
    s = lib.qsa_sparse_attention_splits(64, 16, 2, 128, 2063, 1)
    assert s >= 1 and s & (s - 1) == 0
    assert lib.qsa_sparse_attention_splits(32768, 16, 2, 128, 2063, 0) == 1
    # Decode rows: 64 rows x 2 kv heads take 2 splits (a full round); small
    # batches split up to a round, never past it (36 and 48 rows: 2, not 4;
    # 24 rows: 4, not 8), and keep at least 8 tiles (256 tokens) each.
    assert lib.qsa_sparse_attention_splits(64, 16, 2, 128, 2063, 1) == 2
    assert lib.qsa_sparse_attention_splits(48, 16, 2, 128, 2063, 1) == 2
    assert lib.qsa_sparse_attention_splits(36, 16, 2, 128, 2063, 1) == 2
    assert lib.qsa_sparse_attention_splits(32, 16, 2, 128, 2063, 1) == 4
    assert lib.qsa_sparse_attention_splits(24, 16, 2, 128, 2063, 1) == 4
    assert lib.qsa_sparse_attention_splits(16, 16, 2, 128, 2063, 1) == 8
    assert lib.qsa_sparse_attention_splits(8, 16, 2, 128, 2063, 1) == 8
    assert lib.qsa_sparse_attention_splits(1, 16, 2, 128, 2063, 1) == 8
    assert lib.qsa_sparse_attention_splits(8, 16, 2, 128, 511, 1) == 2   # 16 tiles
    assert lib.qsa_sparse_attention_splits(8, 16, 2, 128, 480, 1) == 1   # 15 tiles


def test_prefill_span_rows():
    """Spans never exceed the logits cap, and are whole rounds of 256 x 32 rows
    when the cap allows one."""
    lib = _lib.load()
    cap = 64 << 20
    assert lib.qsa_indexer_prefill_span_rows(1536, cap) == 8192      # cap 10922 rows
    assert lib.qsa_indexer_prefill_span_rows(64, cap) == 262144      # cap exactly whole rounds
    assert lib.qsa_indexer_prefill_span_rows(6000, cap) == cap // (4 * 6000)  # under one round
    assert lib.qsa_indexer_prefill_span_rows(1 << 30, cap) == 1
    for cols in (64, 100, 1536, 2048, 4099, 32768):
        rows = lib.qsa_indexer_prefill_span_rows(cols, cap)
        assert 1 <= rows and rows * cols * 4 <= cap


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_fastdiv_exhaustive_host(tmp_path):
    src = tmp_path / "fd.cpp"
    src.write_text(r'''
#include "fastdiv.h"
#include <cstdio>
#include <cstdint>
int main() {
  const int32_t divisors[] = {1, 2, 3, 4, 5, 7, 15, 16, 17, 31, 64, 100, 255, 256, 272, 1000,
                              4096, 65535, 65536, 1 << 20, 2147483647};
  uint32_t x = 12345;
  for (int32_t d : divisors) {
    qsa::FastDiv f = qsa::FastDiv::make(d);
    for (int32_t n = 0; n < 200000; ++n)
      if (f.div(n) != n / d) { printf("FAIL d=%d n=%d\n", d, n); return 1; }
    for (int i = 0; i < 200000; ++i) {
      x = x * 1664525u + 1013904223u;
      int32_t n = (int32_t)(x & 0x7fffffffu);
      if (f.div(n) != n / d) { printf("FAIL d=%d n=%d\n", d, n); return 1; }
    }
    int32_t top = 2147483647;
    if (f.div(top) != top / d) { printf("FAIL d=%d top\n", d); return 1; }
  }
  printf("OK\n");
  return 0;
}
''')
    exe = tmp_path / "fd"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "qsa_vllm_amd" / "csrc"),
                    str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and "OK" in out.stdout, out.stdout


TORCH_OPS = ("topk", "topk_expand", "indexer_prepare", "store_cache_rows", "compress_groups",
             "expand_block_indices", "indexer_norm_rope", "indexer_decode", "indexer_prefill",
             "select_decode", "select_prefill", "sparse_attention", "sparse_attention_merge")


def test_torch_op_layer_defines_every_op():
    import torch

    import qsa_vllm_amd.ops  # noqa: F401  (loads libqsa_torch_ops.so)

    ns = torch.ops.yulan_qsa_kernels
    for name in TORCH_OPS:
        assert getattr(ns, name).default._schema.name == f"yulan_qsa_kernels::{name}"
    # the reference schemas, verbatim (ops/csrc/topk.cu:549-552)
    assert str(ns.topk.default._schema) == (
        "yulan_qsa_kernels::topk(Tensor scores, Tensor lengths, Tensor(a!) output) -> ()")
    assert str(ns.topk_expand.default._schema) == (
        "yulan_qsa_kernels::topk_expand(Tensor scores, Tensor lengths, Tensor positions, "
        "Tensor sequence_lengths, Tensor token_to_req, Tensor table, Tensor(a!) output, "
        "Tensor(b!) counts, int ratio, int page_size, bool physical, bool store_counts) -> ()")


def test_torch_ops_reject_host_tensors():
    """No CPU kernel is registered: host tensors are refused before any HIP call."""
    import torch

    import qsa_vllm_amd.ops  # noqa: F401

    scores = torch.zeros(2, 8)
    with pytest.raises((RuntimeError, NotImplementedError)):
        torch.ops.yulan_qsa_kernels.topk(scores, torch.zeros(2, dtype=torch.int32),
                                         torch.zeros(2, 4, dtype=torch.int32))


def test_torch_ops_meta_kernels_trace_shapes():
    import torch

    import qsa_vllm_amd.ops  # noqa: F401

    m = dict(device="meta")
    torch.ops.yulan_qsa_kernels.sparse_attention(
        torch.empty(4, 16, 128, dtype=torch.bfloat16, **m),
        torch.empty(8, 16, 2, 128, dtype=torch.bfloat16, **m),
        torch.empty(8, 16, 2, 128, dtype=torch.bfloat16, **m),
        torch.empty(4, 64, dtype=torch.int32, **m), torch.empty(1, 1, dtype=torch.int32, **m),
        torch.empty(4, dtype=torch.int32, **m), torch.empty(4, 16, 128, dtype=torch.bfloat16, **m),
        None, None, True, 0)


def test_decode_select_attention_fusion_rule():
    """Which decode batch shapes the combined selection + attention runs as one
    launch: the top-k's 512-thread shapes (fewer than 1024 rows, at most 2048
    logits columns), an 8-wave attention plan, at most 2 kv heads per
    workgroup."""
    fuses = _lib.load().qsa_decode_select_attention_fuses
    # decode_32k: 64 rows x 2048 columns, 16 q / 2 kv heads x 128, width 2063.
    assert fuses(64, 2048, 2063, 16, 16, 2, 128) == 1
    assert fuses(64, 1024, 2063, 16, 16, 2, 128) == 1
    assert fuses(256, 2048, 2063, 16, 16, 2, 128) == 1  # 2 kv heads per workgroup
    assert fuses(64, 2048, 2063, 16, 8, 1, 64) == 1
    assert fuses(1023, 2048, 2063, 16, 16, 2, 128) == 1
    assert fuses(1024, 2048, 2063, 16, 16, 2, 128) == 0  # throughput-shaped top-k
    # A wide class: the first 2048 columns in the 512 x 4 shape, longer rows
    # selected inside the workgroup, up to 32768 columns.
    assert fuses(64, 4096, 2063, 16, 16, 2, 128) == 1
    assert fuses(64, 32768, 2063, 16, 16, 2, 128) == 1
    assert fuses(64, 32769, 2063, 16, 16, 2, 128) == 0
    assert fuses(64, 65536, 2063, 16, 16, 2, 128) == 0
    # Small batches run 8-wave attention workgroups too, so they fuse.
    assert fuses(16, 2048, 2063, 16, 16, 2, 128) == 1
    assert fuses(1, 1024, 2063, 16, 16, 2, 128) == 1
    assert fuses(8, 8192, 2063, 16, 16, 2, 128) == 1
    assert fuses(512, 2048, 2063, 16, 16, 4, 128) == 0   # 4 kv heads per workgroup
    assert fuses(64, 1024, 16399, 16, 16, 2, 128) == 0   # 1024 blocks need more than the stage
    assert fuses(64, 2048, 2063, 16, 16, 2, 96) == 0
    assert fuses(0, 2048, 2063, 16, 16, 2, 128) == 0


def _select_attend_args(**over):
    a = dict(scores=1 << 20, srs=2048, rows=4, cols=2048, lengths=1 << 21, pos=1 << 22,
             seq=1 << 23, nreq=4, t2r=1 << 24, table=1 << 25, tabr=2048, tabw=2048, ratio=16,
             idx=1 << 26, idxr=2063, width=2063, counts=1 << 27, q=1 << 28, qr=2048, qh=128,
             hq=16, d=128, k=1 << 29, kb=8192, kt=512, kh=128, v=(1 << 29) + 256, vb=8192,
             vt=512, vh=128, nblk=64, page=16, hkv=2, out=1 << 30, outr=2048, outh=128,
             gate=None, gr=0, gh=0, gd=0, splits=1, ws=None, wsb=0, stream=None)
    a.update(over)
    return list(a.values())


def test_decode_select_attention_argument_errors_need_no_launch():
    lib = _lib.load()
    f = lib.qsa_decode_select_attention
    assert f(*_select_attend_args(rows=0)) == 0
    assert f(*_select_attend_args(ratio=0)) == -1
    assert b"ratio" in lib.qsa_last_error()
    assert f(*_select_attend_args(width=8)) == -1                 # topk = 8 / 16 = 0
    assert f(*_select_attend_args(counts=None)) == -1
    assert f(*_select_attend_args(table=None)) == -1
    assert f(*_select_attend_args(d=96)) == -2                    # the attention's checks
    assert f(*_select_attend_args(splits=4)) == -4                # partials need a workspace
    assert lib.qsa_decode_select_attention_workspace_bytes(64, 2048, 2063, 16, 16, 128, 2) == \
        lib.qsa_sparse_attention_workspace_bytes(64, 16, 128, 2)
    # Long rows: the top-k's partition winners may be the larger workspace.
    assert lib.qsa_decode_select_attention_workspace_bytes(2048, 65536, 2063, 16, 16, 128, 1) == \
        lib.qsa_topk_workspace_bytes(2048, 65536, 128)
