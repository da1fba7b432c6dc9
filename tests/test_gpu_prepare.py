"""GPU parity of the indexer preparation kernels against the CPU oracle
(bit-exact: the kernels and the oracle round every step identically)."""

import pytest
import torch

import oracle
from qsa_vllm_amd.ops import IndexerRMSNorm, indexer_norm_rope, qsa_prepare
from qsa_vllm_amd.workloads import make_prepare_case

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _oracle_run(case):
    """oracle.prepare on CPU copies of the case's inputs and outputs."""
    cpu = {k: v.cpu() for k, v in case.clone_outputs().items()}
    args, kwargs = case.call_args()
    args = [a.cpu() if isinstance(a, torch.Tensor) else a for a in args]
    from types import SimpleNamespace
    args[6] = SimpleNamespace(**{k: v.cpu() for k, v in vars(case.raw).items()})
    args[7] = SimpleNamespace(**{k: v.cpu() for k, v in vars(case.comp).items()})
    d = case.main_key.shape[2]
    args[8], args[9] = cpu["state_cache"], cpu["compressed_cache"]
    args[12], args[13] = cpu["main_kv"][..., :d], cpu["main_kv"][..., d:]
    query = oracle.prepare(*args, **kwargs)
    return query, cpu


def _check(case):
    want_q, want = _oracle_run(case)
    print(f"prepare tokens={case.index_qk.shape[0]} heads={case.num_index_heads} "
          f"dim={case.index_head_dim} ratio={case.compress_ratio} "
          f"state={case.state_cache.shape[1]} rotary={case.rotary_dim}", flush=True)
    args, kwargs = case.call_args()
    got_q = qsa_prepare(*args, **kwargs)
    torch.cuda.synchronize()
    assert torch.equal(got_q.cpu(), want_q)
    assert torch.equal(case.state_cache.cpu(), want["state_cache"])
    assert torch.equal(case.compressed_cache.cpu(), want["compressed_cache"])
    assert torch.equal(case.main_kv.cpu(), want["main_kv"])


@pytest.mark.parametrize("prefix,chunk,kw", [
    # decode steps: one token per request, some closing a group
    ([15, 31, 100, 7, 47], [1, 1, 1, 1, 1], dict()),
    # chunked prefill: chunks starting mid-group read the ring
    ([5, 16, 0], [40, 17, 33], dict()),
    ([5, 16, 0], [40, 17, 33], dict(state_size=32)),
    # small heads, 64 dims, other ratios and rotary widths
    ([6, 0, 13, 2], [3, 9, 1, 30], dict(num_index_heads=4, index_head_dim=64, compress_ratio=4,
                                        rotary_dim=32, main_kv_heads=1, main_head_dim=64)),
    ([6, 0, 13], [3, 9, 21], dict(num_index_heads=3, index_head_dim=64, compress_ratio=8,
                                  rotary_dim=64, main_kv_heads=4, main_head_dim=64)),
    ([6, 0, 13], [3, 9, 21], dict(rotary_dim=0)),
    ([6, 0, 13], [3, 9, 21], dict(rotary_dim=128)),
    # unmapped slots and padding work items
    ([5, 8], [12, 9], dict(drop_slot_every=3, work_pad=20)),
])
def test_prepare_parity(prefix, chunk, kw):
    case = make_prepare_case(prefix, chunk, device=DEV, seed=len(prefix) * 7 + sum(chunk), **kw)
    _check(case)


@pytest.mark.parametrize("seed", range(16))
def test_prepare_random_cases(seed):
    """Seeded random batches: request counts, prefixes (mid-group and past the
    ring), chunk lengths, index-head counts that leave partial 8-row groups,
    64/128 dims, ratios, rotary widths, ring sizes, kv heads, unmapped slots."""
    g = torch.Generator().manual_seed(3000 + seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=g))]  # noqa: E731
    nreq = pick([1, 2, 4, 6])
    prefix = torch.randint(0, 300, (nreq,), generator=g).tolist()
    chunk = torch.randint(1, 80, (nreq,), generator=g).tolist()
    dim = pick([64, 128])
    ratio = pick([4, 8, 16])
    kw = dict(num_index_heads=pick([1, 3, 8, 16, 32]), index_head_dim=dim, compress_ratio=ratio,
              rotary_dim=pick([0, 32, 64, dim]), state_size=pick([None, 2 * ratio]),
              main_kv_heads=pick([1, 2, 4]), main_head_dim=dim, drop_slot_every=pick([0, 5]))
    case = make_prepare_case(prefix, chunk, device=DEV, seed=seed, **kw)
    _check(case)


def test_prepare_parity_prefill_8k_on_16k():
    # The benchmark's chunked prefill: 4 requests x 8192 tokens on a 16384 prefix.
    case = make_prepare_case([16384] * 4, [8192] * 4, device=DEV, seed=1)
    _check(case)


def test_prepare_graph_replay_equals_eager():
    case = make_prepare_case([5, 16, 0], [40, 17, 33], device=DEV, seed=3)
    start = case.clone_outputs()
    args, kwargs = case.call_args()

    def reset():
        case.state_cache.copy_(start["state_cache"])
        case.compressed_cache.copy_(start["compressed_cache"])
        case.main_kv.copy_(start["main_kv"])

    eager_q = qsa_prepare(*args, **kwargs)
    eager = case.clone_outputs()
    reset()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        qsa_prepare(*args, **kwargs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graph_q = qsa_prepare(*args, **kwargs)
    for _ in range(3):
        reset()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(graph_q, eager_q)
        for k, v in case.clone_outputs().items():
            assert torch.equal(v, eager[k]), k


@pytest.mark.parametrize("dim,rotary", [(128, 64), (64, 32), (128, 0), (64, 64)])
def test_norm_rope_parity(dim, rotary):
    g = torch.Generator().manual_seed(dim + rotary)
    tokens, heads = 37, 5
    base = (torch.randn(tokens, heads + 2, dim + 16, generator=g) * 1.5).to(torch.bfloat16)
    values = base[:, 1:heads + 1, 8:8 + dim]            # strided view, unit dim stride
    positions = torch.randint(-2, 70, (tokens,), generator=g)  # some outside the table
    table = oracle.rotary_cache_table(64, rotary, 1.0e7) if rotary else torch.zeros(64, 0,
                                                                                    dtype=torch.bfloat16)
    norm = IndexerRMSNorm(dim, 1e-6)
    norm.weight.data = (1.0 + 0.3 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    want = oracle.norm_rope(values, positions.repeat_interleave(heads), norm.weight.data, table,
                            1e-6, rotary).view(tokens, heads, dim)
    norm = norm.to(DEV)
    values_dev = base.to(DEV)[:, 1:heads + 1, 8:8 + dim]
    got = indexer_norm_rope(values_dev, norm, positions.to(DEV), table.contiguous().to(DEV), rotary)
    assert torch.equal(got.cpu(), want)
