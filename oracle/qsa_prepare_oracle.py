"""CPU restatement of the indexer preparation (the producers of the path).

TEST INFRASTRUCTURE ONLY: what ``qsa_indexer_prepare`` and
``qsa_indexer_norm_rope`` are tested against. Nothing under ``qsa_vllm_amd`` imports it.

Follows ops/normalization.py:17-83 and ops/prepare.py:16-225 of the reference
plugin. Arithmetic, step by step as the reference rounds it (it compiles with
``enable_fp_fusion=False``):

* the sum of squares of a row's bf16 values is formed exactly and rounded
  once to fp32; ``inv = 1 / sqrt(fp32(sum) / dim + eps)`` is evaluated in
  double and rounded to fp32 (the correctly rounded value - the reference's
  fp32 tree sum and approximate ``rsqrt`` may differ from it in the last fp32
  bits, which moves a bf16 output by one unit only when it lies that close to
  a rounding boundary);
* ``scaled = bf16(bf16(x * inv) * gamma)`` with fp32 products;
* rotate-half RoPE on the first ``rotary`` dims:
  ``bf16(bf16(scaled * cos) + bf16(rotated * sin))``, ``rotated`` the partner
  dim (d +/- rotary/2), negated in the first half; cos/sin from the bf16
  table row of the position, zero for positions outside the table;
* compression groups: fp32 sum of the ``ratio`` raw keys in member order,
  divided by ``ratio``, rounded to bf16, then the same norm + RoPE at the
  group's first position.

Pinning (``tests/test_prepare_oracle.py``): a pure-Python scalar statement
(``tests/restate.py``: fp32 rounding by struct, bf16 by bit arithmetic)
bit for bit; closed forms (constant rows, position 0 leaves the row
unrotated, pair norms preserved by the rotation against a double-precision
rotation, the table against cos/sin in double); known-answer vectors in
``tests/golden/qsa_golden.json``.

Parity unpinned: the upstream metadata builder that produces ``k_work``,
ring and compressed slot mappings in serving (vllm 0.30.0, not vendored);
the workloads build them from what this kernel reads.
"""

from __future__ import annotations

import torch

__all__ = ["rotary_cache_table", "norm_rope", "prepare"]


def rotary_cache_table(max_position, rotary_dim, theta):
    """[max_position, rotary_dim] bf16 (cos, then sin) in fp32 steps
    (ops/normalization.py:17-23)."""
    channels = torch.arange(0, rotary_dim, 2, dtype=torch.float32)
    inverse = theta ** (-channels / rotary_dim)
    phases = torch.outer(torch.arange(max_position, dtype=torch.float32), inverse)
    return torch.cat((phases.cos(), phases.sin()), dim=-1).to(torch.bfloat16)


def _bf16(x):
    return x.to(torch.bfloat16).to(torch.float32)


def norm_rope(x, positions, weight, cos_sin, eps, rotary):
    """RMSNorm + partial RoPE of rows x [n, dim] bf16 at positions [n]
    (ops/normalization.py:44-68, ops/prepare.py:17-46). Returns bf16 [n, dim]."""
    x = x.reshape(-1, x.shape[-1]).to(torch.float32)
    n, dim = x.shape
    sumsq = (x.double() * x.double()).sum(-1).to(torch.float32)
    mean = sumsq / torch.tensor(float(dim), dtype=torch.float32)
    inv = (1.0 / torch.sqrt((mean + torch.tensor(eps, dtype=torch.float32)).double())).to(torch.float32)
    scaled = _bf16(_bf16(x * inv[:, None]) * weight.to(torch.float32)[None, :])
    out = scaled.clone()
    if rotary:
        half = rotary // 2
        d = torch.arange(rotary)
        partner = torch.where(d < half, d + half, d - half)
        rotated = scaled[:, partner]
        rotated = torch.where(d[None, :] < half, -rotated, rotated)
        pos = positions.reshape(-1).to(torch.int64)
        ok = (pos >= 0) & (pos < cos_sin.shape[0])
        table = cos_sin.to(torch.float32)[pos.clamp(0, cos_sin.shape[0] - 1)]
        table = torch.where(ok[:, None], table, torch.zeros_like(table))
        channel = d % half
        cos = table[:, channel]
        sin = table[:, half + channel]
        first = _bf16(scaled[:, :rotary] * cos)
        second = _bf16(rotated * sin)
        out[:, :rotary] = _bf16(first + second)
    return out.to(torch.bfloat16)


def prepare(index_qk, positions, q_weight, k_weight, cos_sin, eps, raw, comp, state_cache,
            compressed_cache, main_key, main_value, main_key_cache, main_value_cache, main_slots,
            *, num_index_heads, index_head_dim, rotary_dim, compress_ratio):
    """qsa_prepare on CPU tensors (ops/prepare.py:49-225). Writes the caches in
    place and returns the normalised index queries [tokens, heads, dim] bf16.

    ``raw``: slot_mapping, block_table, query_start_loc, logical_positions;
    ``comp``: slot_mapping, k_work_metadata."""
    heads, dim, R = num_index_heads, index_head_dim, compress_ratio
    tokens = index_qk.shape[0]
    # Index queries (ops/prepare.py:97-118).
    q_rows = index_qk[:, : heads * dim].reshape(tokens * heads, dim)
    q_pos = positions.reshape(-1)[:tokens].repeat_interleave(heads)
    query = norm_rope(q_rows, q_pos, q_weight, cos_sin, eps, rotary_dim).reshape(tokens, heads, dim)
    keys = index_qk[:, heads * dim: (heads + 1) * dim]

    state = state_cache.view(state_cache.shape[0], state_cache.shape[1], -1)
    compressed = compressed_cache.view(compressed_cache.shape[0], compressed_cache.shape[1], -1)
    state_size, comp_page = state.shape[1], compressed.shape[1]
    qsl = raw.query_start_loc.tolist()
    logical = raw.logical_positions.tolist()
    num_requests = len(qsl) - 1
    ring_before = state.clone()  # group reads see the ring before this launch's commits
    commits = []
    # Compression groups, then ring commits (ops/prepare.py:120-174).
    for request, work in comp.k_work_metadata.tolist():
        if request < 0 or request >= num_requests:
            continue
        qs, qe = qsl[request], qsl[request + 1]
        qlen = qe - qs
        if qlen <= 0 or qs < 0 or qe > tokens:
            continue
        chunk_end = logical[qe - 1]
        chunk_start = chunk_end - qlen + 1
        if chunk_start < 0:
            continue
        groups = (chunk_end + 1) // R - chunk_start // R
        block = int(raw.block_table[request, 0])
        ring_ok = 0 <= block < state.shape[0]
        if work < groups:
            first_boundary = ((chunk_start + R) // R) * R - 1
            end = first_boundary + work * R
            boundary_token = qs + end - chunk_start
            if boundary_token >= qe:  # positions inconsistent with the chunk: item skipped
                continue
            acc = torch.zeros(dim, dtype=torch.float32)
            for m in range(R):
                src = end - (R - 1) + m
                if src >= chunk_start:
                    row = keys[qs + src - chunk_start]
                elif ring_ok:
                    row = ring_before[block, src % state_size]
                else:
                    row = torch.zeros(dim, dtype=torch.bfloat16)
                acc = acc + row.to(torch.float32)  # member order, fp32
            pooled = (acc / torch.tensor(float(R), dtype=torch.float32)).to(torch.bfloat16)
            out = norm_rope(pooled[None], torch.tensor([end - (R - 1)]), k_weight, cos_sin, eps,
                            rotary_dim)[0]
            slot = int(comp.slot_mapping[boundary_token])
            if slot >= 0 and slot // comp_page < compressed.shape[0]:
                compressed[slot // comp_page, slot % comp_page] = out
        if work == 0:
            suffix = min(qlen, state_size)
            for off in range(suffix):
                token = qe - suffix + off
                slot = int(raw.slot_mapping[token])
                if slot >= 0 and slot // state_size < state.shape[0]:
                    commits.append((slot, token))
    for slot, token in commits:
        state[slot // state_size, slot % state_size] = keys[token]
    # Main K/V slot writes (ops/prepare.py:74-95).
    page = main_key_cache.shape[1]
    for token, slot in enumerate(main_slots.tolist()[:tokens]):
        if slot < 0 or slot // page >= main_key_cache.shape[0]:
            continue
        main_key_cache[slot // page, slot % page] = main_key[token]
        main_value_cache[slot // page, slot % page] = main_value[token]
    return query
