"""Writes qsa_golden.json: small known-answer vectors for the QSA path.

The reference plugin ships no test vectors, so these are computed here from
the pure-Python statements in tests/restate.py (rank counting, column-wise
expansion, scalar-loop scores and attention in double precision, scalar
RMSNorm + RoPE and group pooling with emulated fp32/bf16 rounding), from
inputs chosen so that every value is exact in bf16. The file freezes the
expected answers: the oracle and the GPU kernels are both checked against it.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import math
import random
import struct
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from tests import restate  # noqa: E402

OUT = Path(__file__).with_name("qsa_golden.json")


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def topk_cases(rng):
    cases = []
    specials = [0.0, -0.0, 1.0, -1.0, 2.5, float("inf"), -float("inf"), 1e-39, -1e-39]
    for n, k, mode in [(12, 4, "specials"), (40, 8, "ties"), (64, 16, "random"), (5, 8, "short"),
                       (33, 32, "random")]:
        if mode == "specials":
            bits = [f32_bits(rng.choice(specials)) for _ in range(n)]
            bits[3] = 0x7FC00000          # positive quiet NaN: above +inf as uint32
            bits[7] = 0xFFC00000          # negative quiet NaN: the largest key
        elif mode == "ties":
            bits = [f32_bits(float(rng.randint(0, 3))) for _ in range(n)]
        else:
            bits = [f32_bits(rng.uniform(-4.0, 4.0)) for _ in range(n)]
        length = n if mode != "short" else 3
        want = restate.topk_by_rank(bits, length, k)
        cases.append({"bits": bits, "length": length, "k": k, "ids": want})
    return cases


def expand_cases(rng):
    cases = []
    for ratio, page, physical in [(4, 8, True), (4, 6, True), (4, 4, False), (16, 16, True)]:
        k = 3
        width = k * ratio + ratio - 1
        seq_lens = [rng.randint(ratio * 2, ratio * 9) for _ in range(3)]
        table_w = max(seq_lens) // page + 2
        table = [[rng.randint(0, 60) for _ in range(table_w)] for _ in range(3)]
        table[1][0] = -1
        rows = []
        for r, req in enumerate([0, 1, 2, -1]):
            sl = seq_lens[req] if req >= 0 else 10
            pos = sl - 1 if r != 2 else sl // 2
            nblk = rng.randint(k + 2, k + 6)
            scores = [rng.uniform(0.0, 3.0) for _ in range(nblk)]
            lengths = min(nblk, (pos + 1) // ratio, (seq_lens[req] if req >= 0 else 0) // ratio)
            lengths = max(lengths, 0)
            bits = [f32_bits(x) for x in scores]
            ids = restate.topk_by_rank(bits, lengths, k)
            row, count = restate.expand_columns([i for i in ids], pos, req, seq_lens, ratio,
                                                width, physical, table, page)
            rows.append({"bits": bits, "length": lengths, "position": pos, "request": req,
                         "out": row, "count": count})
        cases.append({"ratio": ratio, "page": page, "physical": physical, "width": width,
                      "seq_lens": seq_lens, "table": table, "rows": rows})
    return cases


def bf16_exact(rng, n, scale=8):
    # Multiples of 1/scale in [-2, 2]: exact in bf16, and products/sums of a
    # few of them are exact in fp32, so the expected scores are exact.
    return [rng.randint(-2 * scale, 2 * scale) / scale for _ in range(n)]


def indexer_cases(rng):
    heads, dim, npages, cpage = 4, 64, 3, 16
    q = [[bf16_exact(rng, dim) for _ in range(heads)] for _ in range(2)]
    cache = [[bf16_exact(rng, dim) for _ in range(cpage)] for _ in range(npages)]
    table = [[2, 0], [1, 2]]
    visible = [20, 9]
    scores = []
    for r in range(2):
        keys = [cache[table[r][c // cpage]][c % cpage] for c in range(visible[r])]
        scores.append(restate.relu_head_scores(q[r], keys))
    return {"heads": heads, "dim": dim, "cache_page": cpage, "q": q, "cache": cache,
            "table": table, "visible": visible, "scores": scores}


def attention_case(rng):
    hq, hkv, dim, page, nblk = 4, 2, 64, 4, 6
    group = hq // hkv
    k = [[[bf16_exact(rng, dim, 4) for _ in range(hkv)] for _ in range(page)] for _ in range(nblk)]
    v = [[[bf16_exact(rng, dim, 4) for _ in range(hkv)] for _ in range(page)] for _ in range(nblk)]
    q = [[bf16_exact(rng, dim, 4) for _ in range(hq)] for _ in range(2)]
    # physical slots (block * page + offset); -1 and an out-of-cache slot are invalid
    indices = [[0, 5, 9, 22, -1, 13], [7, 7, nblk * page + 1, 2, 3, -1]]
    counts = [6, 4]
    out = []
    for r in range(2):
        valid = [s for s in indices[r][:counts[r]] if 0 <= s < nblk * page]
        rows = []
        for h in range(hq):
            g = h // group
            keys = [k[s // page][s % page][g] for s in valid]
            vals = [v[s // page][s % page][g] for s in valid]
            rows.append(restate.softmax_attend(q[r][h], keys, vals) if keys else [0.0] * dim)
        out.append(rows)
    return {"hq": hq, "hkv": hkv, "dim": dim, "page": page, "blocks": nblk, "q": q, "k": k,
            "v": v, "indices": indices, "counts": counts, "out": out}


def bf16_table(positions, rotary, theta):
    # cos/sin table rounded to bf16 from double precision (input data only).
    half = rotary // 2
    rows = []
    for p in range(positions):
        angles = [p * theta ** (-2.0 * c / rotary) for c in range(half)]
        rows.append([restate.bf16(restate.f32(math.cos(a))) for a in angles]
                    + [restate.bf16(restate.f32(math.sin(a))) for a in angles])
    return rows


def norm_rope_case(rng):
    dim, rotary, eps = 64, 32, 1e-6
    table = bf16_table(16, rotary, 1.0e4)
    x = [bf16_exact(rng, dim) for _ in range(4)]
    gamma = [rng.randint(12, 20) / 16 for _ in range(dim)]
    positions = [0, 3, 7, 15]
    out = [restate.norm_rope_row(x[r], positions[r], gamma, table, eps, rotary) for r in range(4)]
    return {"dim": dim, "rotary": rotary, "eps": eps, "table": table, "x": x, "gamma": gamma,
            "positions": positions, "out": out}


def prepare_case(rng):
    """Two requests: prefix 6 + chunk 3 (its first group reads ring members)
    and prefix 0 + chunk 9; ratio 4, ring 4, 2 index heads x 64, 1 main kv
    head x 64, main page 4."""
    heads, dim, ratio, state, rotary, eps = 2, 64, 4, 4, 32, 1e-6
    mdim, mpage, cpage = 64, 4, 4
    prefix, chunk = [6, 0], [3, 9]
    positions = [p for q in range(2) for p in range(prefix[q], prefix[q] + chunk[q])]
    tokens = len(positions)
    qsl = [0, chunk[0], chunk[0] + chunk[1]]
    table = bf16_table(max(positions) + 1, rotary, 1.0e4)
    index_qk = [bf16_exact(rng, (heads + 1) * dim) for _ in range(tokens)]
    main_key = [bf16_exact(rng, mdim) for _ in range(tokens)]
    main_value = [bf16_exact(rng, mdim) for _ in range(tokens)]
    q_gamma = [rng.randint(12, 20) / 16 for _ in range(dim)]
    k_gamma = [rng.randint(12, 20) / 16 for _ in range(dim)]
    ring_blocks = [2, 0]                 # of 3 ring blocks
    state_cache = [[bf16_exact(rng, dim) for _ in range(state)] for _ in range(3)]
    state_slots = [ring_blocks[0 if t < qsl[1] else 1] * state + positions[t] % state
                   for t in range(tokens)]
    comp_pages = [[1], [0, 2]]           # compressed pages of 4 keys
    comp_slots = []
    for t in range(tokens):
        q = 0 if t < qsl[1] else 1
        p = positions[t]
        g = (p + 1) // ratio - 1
        comp_slots.append(comp_pages[q][g // cpage] * cpage + g % cpage if (p + 1) % ratio == 0
                          else -1)
    k_work = [[1, 1], [0, 0], [-1, 0], [1, 0]]
    main_slots = [5, 0, 11, -1, 3, 7, 8, 2, 9, 1, 12, 6]
    comp_cache = [[[0.0] * dim for _ in range(cpage)] for _ in range(3)]
    main_cache = [[[0.0] * (2 * mdim) for _ in range(mpage)] for _ in range(4)]
    # expected results
    query = [[restate.norm_rope_row(index_qk[t][h * dim:(h + 1) * dim], positions[t], q_gamma,
                                    table, eps, rotary) for h in range(heads)] for t in range(tokens)]
    state_after = [[list(r) for r in blk] for blk in state_cache]
    comp_after = [[list(r) for r in pg] for pg in comp_cache]
    for q in range(2):
        toks = list(range(qsl[q], qsl[q + 1]))
        ring = {s: state_cache[ring_blocks[q]][s] for s in range(state)}
        groups, after = restate.prepare_request([positions[t] for t in toks],
                                                [index_qk[t][heads * dim:] for t in toks], ring,
                                                ratio, state, k_gamma, table, eps, rotary)
        for t in toks:
            if comp_slots[t] >= 0:
                comp_after[comp_slots[t] // cpage][comp_slots[t] % cpage] = groups[positions[t]]
        for s in range(state):
            state_after[ring_blocks[q]][s] = after[s]
    main_after = [[list(r) for r in pg] for pg in main_cache]
    for t, slot in enumerate(main_slots):
        if slot >= 0:
            main_after[slot // mpage][slot % mpage] = main_key[t] + main_value[t]
    return {"heads": heads, "dim": dim, "ratio": ratio, "state": state, "rotary": rotary,
            "eps": eps, "main_dim": mdim, "main_page": mpage, "comp_page": cpage,
            "positions": positions, "query_start_loc": qsl, "table": table,
            "index_qk": index_qk, "main_key": main_key, "main_value": main_value,
            "q_gamma": q_gamma, "k_gamma": k_gamma, "state_table": [[b] for b in ring_blocks],
            "state_cache": state_cache, "state_slots": state_slots, "comp_slots": comp_slots,
            "k_work": k_work, "main_slots": main_slots, "comp_cache": comp_cache,
            "main_cache": main_cache, "query": query, "state_after": state_after,
            "comp_after": comp_after, "main_after": main_after}


def main():
    rng = random.Random(20261201)
    data = {
        "about": "known answers from tests/restate.py; see tests/golden/make_golden.py",
        "topk": topk_cases(rng),
        "topk_expand": expand_cases(rng),
        "indexer": indexer_cases(rng),
        "attention": attention_case(rng),
        "norm_rope": norm_rope_case(rng),
        "prepare": prepare_case(rng),
    }
    OUT.write_text(json.dumps(data, indent=None, separators=(",", ":")) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
