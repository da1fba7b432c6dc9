"""CPU pins of the prepare oracle (oracle/qsa_prepare_oracle.py): a scalar
statement with emulated rounding, closed forms, and the product's rotary table."""

import math

import pytest
import torch

import oracle
from qsa_vllm_amd.ops.normalization import rotary_cache
from qsa_vllm_amd.workloads import make_prepare_case
from tests import restate


def _rows(n, dim, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, dim, generator=g) * scale).to(torch.bfloat16)


def _gamma(dim, seed):
    g = torch.Generator().manual_seed(seed + 1000)
    return (1.0 + 0.3 * torch.randn(dim, generator=g)).to(torch.bfloat16)


@pytest.mark.parametrize("dim,rotary", [(64, 0), (64, 32), (64, 64), (128, 64), (128, 128)])
def test_norm_rope_matches_scalar_statement(dim, rotary):
    table = oracle.rotary_cache_table(40, rotary, 1.0e7) if rotary else torch.zeros(40, 0)
    x = _rows(7, dim, seed=dim + rotary, scale=2.0)
    gamma = _gamma(dim, dim)
    pos = torch.tensor([0, 1, 5, 17, 39, -1, 40])  # the last two are outside the table
    got = oracle.norm_rope(x, pos, gamma, table.to(torch.bfloat16), 1e-6, rotary)
    tab = table.float().tolist()
    for r in range(x.shape[0]):
        want = restate.norm_rope_row(x[r].float().tolist(), int(pos[r]), gamma.float().tolist(),
                                     tab, 1e-6, rotary)
        assert got[r].float().tolist() == want, r


def test_unit_rms_rows_reduce_to_gamma():
    # Rows of +-1 have mean square 1: inv = 1/sqrt(1 + eps) rounds x back to
    # itself in bf16, so the output is bf16(x * gamma); position 0 rotates by 0.
    g = torch.Generator().manual_seed(3)
    x = (torch.randint(0, 2, (5, 128), generator=g) * 2 - 1).to(torch.bfloat16)
    gamma = _gamma(128, 3)
    want = (x.float() * gamma.float()).to(torch.bfloat16)
    table = oracle.rotary_cache_table(4, 64, 1.0e7)
    got = oracle.norm_rope(x, torch.zeros(5, dtype=torch.int64), gamma, table, 1e-6, 64)
    assert torch.equal(got, want)


def test_position_zero_leaves_rows_unrotated():
    x = _rows(6, 128, seed=11)
    gamma = _gamma(128, 11)
    table = oracle.rotary_cache_table(8, 64, 1.0e7)
    zero = torch.zeros(6, dtype=torch.int64)
    assert torch.equal(oracle.norm_rope(x, zero, gamma, table, 1e-6, 64),
                       oracle.norm_rope(x, zero, gamma, table, 1e-6, 0))


def test_rotation_against_double_precision():
    x = _rows(16, 128, seed=5)
    gamma = _gamma(128, 5)
    theta, rot = 1.0e4, 64
    table = oracle.rotary_cache_table(1000, rot, theta)
    pos = torch.randint(0, 1000, (16,), generator=torch.Generator().manual_seed(9))
    got = oracle.norm_rope(x, pos, gamma, table, 1e-6, rot).double()
    scaled = oracle.norm_rope(x, pos, gamma, table, 1e-6, 0).double()
    half = rot // 2
    for r in range(16):
        p = int(pos[r])
        for d in range(half):
            angle = p * theta ** (-2.0 * d / rot)
            a, b = scaled[r, d].item(), scaled[r, d + half].item()
            want_a = a * math.cos(angle) - b * math.sin(angle)
            want_b = b * math.cos(angle) + a * math.sin(angle)
            tol = 0.02 * (abs(a) + abs(b)) + 1e-6
            assert abs(got[r, d].item() - want_a) <= tol
            assert abs(got[r, d + half].item() - want_b) <= tol
        # dims past the rotary part are the normalised, scaled row
        assert torch.equal(got[r, rot:], scaled[r, rot:])


def test_rotary_table_closed_form():
    rot, theta = 64, 1.0e7
    table = oracle.rotary_cache_table(64, rot, theta).double()
    for p in range(64):
        for c in range(rot // 2):
            angle = p * theta ** (-2.0 * c / rot)
            assert abs(table[p, c].item() - math.cos(angle)) <= 2 ** -8 + 1e-4 * p
            assert abs(table[p, rot // 2 + c].item() - math.sin(angle)) <= 2 ** -8 + 1e-4 * p


def test_product_rotary_cache_matches_oracle_table():
    assert torch.equal(rotary_cache(300, 64, 1.0e7, "cpu"), oracle.rotary_cache_table(300, 64, 1.0e7))


def _run_oracle(case):
    outs = case.clone_outputs()
    args, kwargs = case.call_args()
    args = list(args)
    args[8] = outs["state_cache"]
    args[9] = outs["compressed_cache"]
    kv = outs["main_kv"]
    d = case.main_key.shape[2]
    args[12], args[13] = kv[..., :d], kv[..., d:]
    query = oracle.prepare(*args, **kwargs)
    return query, outs


@pytest.mark.parametrize("prefix,chunk,ratio,state", [
    ([6, 0, 13], [3, 9, 1], 4, 4),      # ring members, group-less request, decode token
    ([9, 30], [11, 2], 4, 8),           # ring larger than the ratio
    ([16, 3], [16, 13], 8, 8),
])
def test_prepare_matches_scalar_statement(prefix, chunk, ratio, state):
    case = make_prepare_case(prefix, chunk, num_index_heads=2, index_head_dim=64,
                             compress_ratio=ratio, state_size=state, rotary_dim=32,
                             main_kv_heads=1, main_head_dim=64, seed=len(prefix) + ratio)
    query, outs = _run_oracle(case)
    dim, heads = 64, 2
    table = case.cos_sin.float().tolist()
    kg = case.k_norm_weight.float().tolist()
    qg = case.q_norm_weight.float().tolist()
    qsl = case.raw.query_start_loc.tolist()
    comp = outs["compressed_cache"].view(-1, dim)
    ring_after = outs["state_cache"]
    for q in range(len(chunk)):
        toks = range(qsl[q], qsl[q + 1])
        positions = [int(case.positions[t]) for t in toks]
        keys = [case.index_qk[t, heads * dim:].float().tolist() for t in toks]
        block = int(case.raw.block_table[q, 0])
        ring = {s: case.state_cache[block, s].float().tolist() for s in range(state)}
        groups, after = restate.prepare_request(positions, keys, ring, ratio, state, kg, table,
                                                1e-6, 32)
        for t, p in zip(toks, positions):
            slot = int(case.comp.slot_mapping[t])
            if (p + 1) % ratio == 0:
                assert comp[slot].float().tolist() == groups[p], (q, p)
            for h in range(heads):
                want = restate.norm_rope_row(case.index_qk[t, h * dim:(h + 1) * dim].float().tolist(),
                                             p, qg, table, 1e-6, 32)
                assert query[t, h].float().tolist() == want
        for s in range(state):
            assert ring_after[block, s].float().tolist() == after[s], (q, s)
    # main K/V rows land at their slots
    kv = outs["main_kv"]
    page = kv.shape[1]
    for t, slot in enumerate(case.main_slots.tolist()):
        assert torch.equal(kv[slot // page, slot % page, :, :64], case.main_key[t])
        assert torch.equal(kv[slot // page, slot % page, :, 64:], case.main_value[t])


def test_prepare_skips_unmapped_slots_and_padding():
    case = make_prepare_case([5, 8], [12, 9], num_index_heads=2, index_head_dim=64,
                             compress_ratio=4, state_size=4, rotary_dim=32, main_kv_heads=1,
                             main_head_dim=64, drop_slot_every=3, work_pad=5, seed=2)
    before = case.clone_outputs()
    _, outs = _run_oracle(case)
    kv0, kv1 = before["main_kv"], outs["main_kv"]
    page = kv0.shape[1]
    written = set()
    for slot in case.main_slots.tolist():
        if slot >= 0:
            written.add((slot // page, slot % page))
    for b in range(kv0.shape[0]):
        for o in range(page):
            if (b, o) not in written:
                assert torch.equal(kv0[b, o], kv1[b, o])
    # compressed rows change only at mapped group slots
    comp0 = before["compressed_cache"].view(-1, 64)
    comp1 = outs["compressed_cache"].view(-1, 64)
    mapped = {s for s in case.comp.slot_mapping.tolist() if s >= 0}
    for s in range(comp0.shape[0]):
        if s not in mapped:
            assert torch.equal(comp0[s], comp1[s])
