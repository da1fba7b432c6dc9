"""Every oracle function is pinned: a deliberately broken copy fails its pin.

Each mutant below is one plausible mistake planted in the oracle's own source
(a dropped term, a wrong sign, index or operand order, a mis-sliced table),
compiled into a fresh module on the CPU. The oracle names the tests use are
pointed at the broken module, and every listed pin test must then fail. A
coverage check requires a mutant for every exported oracle function, so a
function with no pin that catches a mistake cannot hide. The oracle files on
disk are never modified.
"""

from __future__ import annotations

import functools
import sys
import types
from pathlib import Path

import pytest

import oracle
from tests import test_golden as G
from tests import test_helpers_oracle as HO
from tests import test_hybrid_oracle as HY
from tests import test_oracle as O
from tests import test_prepare_oracle as P

ORACLE_DIR = Path(__file__).resolve().parents[1] / "oracle"
HYBRID = sys.modules["oracle.hybrid_oracle"]


def _p(fn, **kw):
    return functools.partial(fn, **kw) if kw else fn


# (file, exported function the mistake is in, original text, broken text, pins)
MUTANTS = [
    # -------------------------------------------------------------- qsa_oracle.py
    ("qsa_oracle.py", "visible_blocks", "(query_positions.long() + 1) // compress_ratio",
     "query_positions.long() // compress_ratio", [O.test_visible_blocks_closed_form]),
    ("qsa_oracle.py", "visible_blocks",
     "return torch.where(token_to_req >= 0, visible, torch.zeros_like(visible))",
     "return visible", [O.test_visible_blocks_closed_form]),
    ("qsa_oracle.py", "decode_logits_columns",
     "columns = 32768 if max_seq_len // compress_ratio <= 32768 else 0",
     "columns = 16384 if max_seq_len // compress_ratio <= 16384 else 0",
     [O.test_logits_width_rules]),
    ("qsa_oracle.py", "prefill_logits_width", "return min(max(64, width), columns)",
     "return min(width, columns)", [O.test_logits_width_rules]),
    ("qsa_oracle.py", "prefill_logits_width",
     "width = _cdiv(_cdiv(max_seq_len, compress_ratio), 64) * 64",
     "width = _cdiv(max_seq_len, compress_ratio)", [O.test_logits_width_rules]),
    ("qsa_oracle.py", "indexer_scores_decode", "return dots.clamp_min(0.0).sum(0) * (dim ** -0.5)",
     "return dots.sum(0) * (dim ** -0.5)",
     [_p(O.test_indexer_scores_bruteforce, dql=1), G.test_oracle_indexer_golden]),
    ("qsa_oracle.py", "indexer_scores_decode", "req = r // decode_query_len", "req = r",
     [_p(O.test_indexer_scores_bruteforce, dql=2),
      _p(O.test_select_paged_tokens_mixed_batch_by_rows, physical=False)]),
    ("qsa_oracle.py", "indexer_scores_prefill", "base = int(query_start_loc[0])", "base = 0",
     [O.test_indexer_prefill_matches_decode_rows]),
    ("qsa_oracle.py", "indexer_scores_prefill",
     "pages = page_table[req, (c // page).clamp_max(table_width - 1)].long()\n"
     "            out[r - query_offset",
     "pages = page_table[0, (c // page).clamp_max(table_width - 1)].long()\n"
     "            out[r - query_offset",
     [O.test_indexer_prefill_matches_decode_rows]),
    ("qsa_oracle.py", "uint32_keys", "return scores.contiguous().view(torch.int32).long() & 0xFFFFFFFF",
     "return scores.contiguous().view(torch.int32).long()",
     [_p(O.test_topk_known_answers, scores=[-1.0, 2.0, 7.0], k=1, expected=[0])]),
    ("qsa_oracle.py", "topk_ids", "order = torch.sort(-keys, stable=True).indices[:k]",
     "order = (length - 1) - torch.sort(-keys.flip(0), stable=True).indices[:k]",
     [O.test_topk_matches_rank_counting,
      _p(O.test_topk_known_answers, scores=[1.0, 3.0, 3.0, 2.0, 3.0], k=2, expected=[1, 2])]),
    ("qsa_oracle.py", "topk_expand", "k = output_width // ratio\n    ids = topk_ids",
     "k = (output_width + 1) // ratio\n    ids = topk_ids",
     [_p(O.test_topk_expand_matches_columnwise_statement, physical=False)]),
    ("qsa_oracle.py", "expand_blocks",
     "counts = torch.minimum(expanded + tail_count, seq_len).to(torch.int32)",
     "counts = (expanded + tail_count).to(torch.int32)",
     [_p(O.test_topk_expand_matches_columnwise_statement, physical=False),
      HO.test_expand_blocks_matches_triton_twin_statement]),
    ("qsa_oracle.py", "expand_blocks", "        valid &= physical_page >= 0\n", "",
     [_p(O.test_topk_expand_matches_columnwise_statement, physical=True),
      HO.test_expand_blocks_matches_triton_twin_statement]),
    ("qsa_oracle.py", "expand_blocks", "tail_start = (p1 // ratio) * ratio",
     "tail_start = (pos // ratio) * ratio",
     [_p(O.test_topk_expand_matches_columnwise_statement, physical=False),
      _p(O.test_topk_expand_matches_columnwise_statement, physical=True)]),
    ("qsa_oracle.py", "store_cache_rows", "cache[slot // page, slot % page, 0, :width] = rows[r, :width]",
     "cache[slot % cache.shape[0], slot // cache.shape[0], 0, :width] = rows[r, :width]",
     [HO.test_store_cache_rows_closed_form]),
    ("qsa_oracle.py", "compress_groups", "position = end - (ratio - 1) + m",
     "position = end - ratio + m", [HO.test_compress_groups_matches_position_walk]),
    ("qsa_oracle.py", "compress_groups",
     "pooled[row, 0] = acc / torch.tensor(float(ratio), dtype=torch.float32)",
     "pooled[row, 0] = acc / torch.tensor(float(ratio - 1), dtype=torch.float32)",
     [HO.test_compress_groups_matches_position_walk]),
    ("qsa_oracle.py", "select_paged_tokens",
     "logits = indexer_scores_prefill(q[num_decode_tokens:], kc, page_table[num_decodes:],",
     "logits = indexer_scores_prefill(q[num_decode_tokens:], kc, page_table,",
     [_p(O.test_select_paged_tokens_mixed_batch_by_rows, physical=False)]),
    ("qsa_oracle.py", "select_paged_tokens",
     "                                        query_start_loc[num_decodes:],",
     "                                        query_start_loc,",
     [_p(O.test_select_paged_tokens_mixed_batch_by_rows, physical=True)]),
    ("qsa_oracle.py", "select_paged_tokens",
     "visible[:num_decode_tokens], decode_query_len, columns)",
     "visible[:num_decode_tokens], 1, columns)",
     [_p(O.test_select_paged_tokens_mixed_batch_by_rows, physical=False)]),
    ("qsa_oracle.py", "sparse_attention", "    scale = dim ** -0.5\n    for r in range(rows):",
     "    scale = dim ** -1.0\n    for r in range(rows):",
     [O.test_attention_dense_causal_equals_sdpa, O.test_attention_bruteforce_loops_physical]),
    ("qsa_oracle.py", "sparse_attention",
     "            qg = q[r, g * group:(g + 1) * group].float()\n            s = (qg",
     "            qg = q[r, g::num_kv_heads].float()\n            s = (qg",
     [O.test_attention_dense_causal_equals_sdpa]),
    ("qsa_oracle.py", "sparse_attention", "valid = (tok >= 0) & (physical_page < num_blocks)",
     "valid = physical_page < num_blocks",
     [O.test_attention_bruteforce_loops_physical]),
    ("qsa_oracle.py", "sparse_attention_partials", "scale_log2 = dim ** -0.5 * 1.4426950408889634",
     "scale_log2 = dim ** -0.5", [O.test_split_merge_identity]),
    ("qsa_oracle.py", "sparse_attention_partials",
     "hi = min(n, ((s + 1) * tiles // num_splits) * block_n)",
     "hi = min(n, ((s + 1) * tiles // num_splits) * block_n - 1)", [O.test_split_merge_identity]),
    ("qsa_oracle.py", "merge_splits", "weights = torch.exp2(shifted)", "weights = torch.exp(shifted)",
     [O.test_split_merge_identity]),
    ("qsa_oracle.py", "decode_step",
     "output_gate=output_gate, indices_are_physical=True,",
     "output_gate=output_gate, indices_are_physical=False,",
     [O.test_decode_step_against_loops]),
    ("qsa_oracle.py", "decode_step", "main_block_table=block_table, main_page_size=k_cache.shape[1])",
     "main_block_table=block_table, main_page_size=1)", [O.test_decode_step_against_loops]),
    # ---------------------------------------------------------- qsa_prepare_oracle.py
    ("qsa_prepare_oracle.py", "rotary_cache_table", "inverse = theta ** (-channels / rotary_dim)",
     "inverse = theta ** (-channels / (rotary_dim // 2))",
     [P.test_rotary_table_closed_form, P.test_product_rotary_cache_matches_oracle_table]),
    ("qsa_prepare_oracle.py", "rotary_cache_table",
     "return torch.cat((phases.cos(), phases.sin()), dim=-1).to(torch.bfloat16)",
     "return torch.cat((phases.sin(), phases.cos()), dim=-1).to(torch.bfloat16)",
     [P.test_rotary_table_closed_form]),
    ("qsa_prepare_oracle.py", "norm_rope",
     "rotated = torch.where(d[None, :] < half, -rotated, rotated)",
     "rotated = torch.where(d[None, :] < half, rotated, -rotated)",
     [_p(P.test_norm_rope_matches_scalar_statement, dim=64, rotary=64),
      P.test_rotation_against_double_precision]),
    ("qsa_prepare_oracle.py", "norm_rope", "sin = table[:, half + channel]", "sin = table[:, channel]",
     [_p(P.test_norm_rope_matches_scalar_statement, dim=128, rotary=64)]),
    ("qsa_prepare_oracle.py", "norm_rope",
     "mean = sumsq / torch.tensor(float(dim), dtype=torch.float32)",
     "mean = sumsq / torch.tensor(float(dim - 1), dtype=torch.float32)",
     [P.test_unit_rms_rows_reduce_to_gamma,
      _p(P.test_norm_rope_matches_scalar_statement, dim=64, rotary=0)]),
    ("qsa_prepare_oracle.py", "prepare",
     "pooled = (acc / torch.tensor(float(R), dtype=torch.float32)).to(torch.bfloat16)",
     "pooled = (acc / torch.tensor(float(R + 1), dtype=torch.float32)).to(torch.bfloat16)",
     [_p(P.test_prepare_matches_scalar_statement, prefix=[0, 5, 31], chunk=[40, 11, 1],
         ratio=4, state=8)]),
    ("qsa_prepare_oracle.py", "prepare", "                src = end - (R - 1) + m",
     "                src = end - R + m",
     [_p(P.test_prepare_matches_scalar_statement, prefix=[0, 5, 31], chunk=[40, 11, 1],
         ratio=4, state=8)]),
    ("qsa_prepare_oracle.py", "prepare", "                if src >= chunk_start:",
     "                if src > chunk_start:",
     [_p(P.test_prepare_matches_scalar_statement, prefix=[0, 5, 31], chunk=[40, 11, 1],
         ratio=4, state=8)]),
    # --------------------------------------------------------------- hybrid_oracle.py
    ("hybrid_oracle.py", "bf16", "return x.to(torch.bfloat16)", "return x.to(torch.float16)",
     [HY.test_bf16_rounds_to_nearest_even]),
    ("hybrid_oracle.py", "rms_norm", "inv = 1.0 / torch.sqrt((xf * xf).mean(-1, keepdim=True) + eps)",
     "inv = 1.0 / torch.sqrt((xf * xf).sum(-1, keepdim=True) + eps)",
     [HY.test_rms_norm_closed_forms]),
    ("hybrid_oracle.py", "rms_norm", "inv = 1.0 / torch.sqrt((xf * xf).mean(-1, keepdim=True) + eps)",
     "inv = 1.0 / torch.sqrt((xf * xf).mean(-1, keepdim=True))",
     [HY.test_rms_norm_zero_row_is_zero]),
    ("hybrid_oracle.py", "gated_norm",
     "gated = bf16(n.double() * bf16(torch.sigmoid(up.double())).double())",
     "gated = bf16(n.double() * bf16(F.silu(up.double())).double())",
     [_p(HY.test_gated_norm_zero_gate_weights, with_residual=False)]),
    ("hybrid_oracle.py", "gated_norm",
     "up = bf16(bf16(F.silu(down.double())).double() @ gate_up.double().T + gate_up_bias.double())",
     "up = bf16(down.double() @ gate_up.double().T + gate_up_bias.double())",
     [HY.test_gated_norm_rank_one_gate_scalar_loops]),
    ("hybrid_oracle.py", "gated_norm", " + gate_up_bias.double())", ")",
     [_p(HY.test_gated_norm_zero_gate_weights, with_residual=False)]),
    ("hybrid_oracle.py", "gated_norm", "        residual = x\n", "",
     [_p(HY.test_gated_norm_zero_gate_weights, with_residual=True)]),
    ("hybrid_oracle.py", "swiglu", "act = bf16(F.silu(gu[:, :i].double()) * gu[:, i:].double())",
     "act = bf16(F.silu(gu[:, i:].double()) * gu[:, :i].double())", [HY.test_swiglu_scalar_loops]),
    ("hybrid_oracle.py", "causal_conv", "out[t] += weight[:, j].double() * padded[t + j]",
     "out[t] += weight[:, K - 1 - j].double() * padded[t + j]",
     [HY.test_causal_conv_matches_conv1d]),
    ("hybrid_oracle.py", "gated_delta_rule", "u = beta[t, h].double() * (v[t, h].double() - kt @ S[h])",
     "u = beta[t, h].double() * v[t, h].double()",
     [HY.test_recurrence_matches_transition_matrices, HY.test_orthonormal_keys_recall_and_overwrite]),
    ("hybrid_oracle.py", "gated_delta_rule", "S[h] *= torch.exp(g[t, h].double())",
     "S[h] *= torch.exp(-g[t, h].double())", [HY.test_no_writes_is_pure_decay]),
    ("hybrid_oracle.py", "gdn_mixer",
     'g = -torch.exp(p["A_log"].double()) * F.softplus(a.double() + p["dt_bias"].double())',
     'g = -torch.exp(p["A_log"].double()) * F.softplus(a.double())',
     [HY.test_gdn_mixer_decay_without_write]),
    ("hybrid_oracle.py", "gdn_mixer",
     "b, a = ba[..., :r].reshape(T, hv), ba[..., r:].reshape(T, hv)",
     "a, b = ba[..., :r].reshape(T, hv), ba[..., r:].reshape(T, hv)",
     [HY.test_gdn_mixer_one_token_from_zero_state]),
    ("hybrid_oracle.py", "gdn_mixer",
     "qs, ks = qs.repeat_interleave(r, 1), ks.repeat_interleave(r, 1)",
     "qs, ks = qs.repeat(1, r, 1), ks.repeat(1, r, 1)",
     [HY.test_gdn_mixer_one_token_from_zero_state]),
    ("hybrid_oracle.py", "gdn_mixer",
     "qs = qs / torch.sqrt((qs * qs).sum(-1, keepdim=True) + 1e-6) * dk ** -0.5",
     "qs = qs / torch.sqrt((qs * qs).sum(-1, keepdim=True) + 1e-6)",
     [HY.test_gdn_mixer_one_token_from_zero_state]),
    ("hybrid_oracle.py", "gdn_mixer",
     'y = bf16(y * p["norm_weight"].double() * F.silu(z.double()))',
     'y = bf16(y * p["norm_weight"].double() * z.double())',
     [HY.test_gdn_mixer_one_token_from_zero_state]),
    ("hybrid_oracle.py", "gdn_mixer",
     "conv, conv_state[slot] = causal_conv(mixed[rows], p[\"conv_weight\"], conv_state[slot])",
     "conv, _ = causal_conv(mixed[rows], p[\"conv_weight\"], conv_state[slot])",
     [HY.test_gdn_mixer_state_hand_off]),
    ("hybrid_oracle.py", "qsa_projection_split",
     "return (qg[..., :head_dim], qg[..., head_dim:], k.reshape",
     "return (qg[..., head_dim:], qg[..., :head_dim], k.reshape",
     [HY.test_qsa_projection_split_index_map]),
]

# Names exported by each oracle file, and where the tests look them up.
_EXPORTS = {
    "qsa_oracle.py": list(sys.modules["oracle.qsa_oracle"].__all__),
    "qsa_prepare_oracle.py": list(sys.modules["oracle.qsa_prepare_oracle"].__all__),
    "hybrid_oracle.py": list(HYBRID.__all__),
}


def _broken_module(file: str, old: str, new: str) -> types.ModuleType:
    src = (ORACLE_DIR / file).read_text()
    assert src.count(old) == 1, f"{file}: the mutated text must occur exactly once: {old!r}"
    mod = types.ModuleType(f"oracle_mutant_{Path(file).stem}")
    exec(compile(src.replace(old, new), f"<mutant of {file}>", "exec"), mod.__dict__)
    return mod


def _point_oracle_at(monkeypatch, file: str, mod: types.ModuleType) -> None:
    for name in _EXPORTS[file]:
        if file == "hybrid_oracle.py":
            monkeypatch.setattr(HYBRID, name, getattr(mod, name))
        else:
            monkeypatch.setattr(oracle, name, getattr(mod, name))


def test_every_exported_oracle_function_has_a_mutant():
    covered = {(file, fn) for file, fn, *_ in MUTANTS}
    missing = [(f, n) for f, names in _EXPORTS.items() for n in names if (f, n) not in covered]
    assert not missing, missing
    for file, fn, *_ in MUTANTS:
        assert fn in _EXPORTS[file], (file, fn)


@pytest.mark.parametrize("case", range(len(MUTANTS)),
                         ids=[f"{m[1]}-{i}" for i, m in enumerate(MUTANTS)])
def test_mutant_fails_its_pins(case, monkeypatch):
    file, fn, old, new, pins = MUTANTS[case]
    assert pins
    mod = _broken_module(file, old, new)
    _point_oracle_at(monkeypatch, file, mod)
    for pin in pins:
        name = getattr(pin, "func", pin).__name__
        # A wrong result fails an assertion; a wrong index may fail first.
        # Errors of the mutant text itself (NameError, SyntaxError) do not count.
        with pytest.raises((AssertionError, IndexError, RuntimeError)):
            pin()
        print(f"{fn}: mutant {case} caught by {name}")
