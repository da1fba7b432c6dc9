"""Independent pure-Python statements used to pin the oracle (tests only).

Each function is written from a different angle than ``oracle/qsa_oracle.py``
(rank counting instead of sorting, column-wise instead of rank-wise expansion,
scalar loops instead of tensor ops) so that a slip in one does not hide in the
other. Sizes must stay tiny.
"""

from __future__ import annotations

import math


def c_div(a, b):
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


def u32_keys(float32_tensor):
    import torch
    return [(v & 0xFFFFFFFF) for v in float32_tensor.contiguous().view(torch.int32).tolist()]


def topk_by_rank(keys, length, k):
    """Selected ids by rank counting: rank(i) = #{key_j > key_i} + #{j < i : key_j == key_i}."""
    if length <= k:
        return [i if i < length else -1 for i in range(k)]
    keys = keys[:length]
    chosen = []
    for i in range(length):
        rank = 0
        for j in range(length):
            if keys[j] > keys[i] or (keys[j] == keys[i] and j < i):
                rank += 1
        if rank < k:
            chosen.append(i)
    assert len(chosen) == k
    return chosen


def expand_columns(block_ids, pos, req, seq_lens, ratio, width, physical, table, page):
    """Column-wise expansion following the reference's second statement of the
    rule (the Triton kernel ``ops/qsa.py:44-106``). Returns (row, count)."""
    k = len(block_ids)
    num_requests = len(seq_lens)
    mapped = 0 <= req < num_requests
    seq_len = seq_lens[req] if mapped else 0
    safe_req = min(max(req, 0), num_requests - 1)
    complete = min(min(c_div(pos + 1, ratio), c_div(seq_len, ratio)), k)
    expanded_count = complete * ratio
    tail_start = c_div(pos + 1, ratio) * ratio
    tail_count = pos + 1 - tail_start
    row = []
    for col in range(width):
        is_exp = col < expanded_count
        rank, off = col // ratio, col % ratio
        block = block_ids[min(rank, k - 1)] if is_exp else -1
        tail_off = col - expanded_count
        is_tail = col >= expanded_count and tail_off < tail_count and tail_off < ratio - 1
        token = block * ratio + off if is_exp else tail_start + tail_off
        valid = (is_exp or is_tail) and 0 <= token < seq_len
        if physical and valid:
            lp = token // page
            pp = table[safe_req][lp] if lp < len(table[safe_req]) else -1
            valid = pp >= 0
            token = pp * page + token % page
        row.append(token if valid else -1)
    count = min(expanded_count + tail_count, seq_len) if mapped else 0
    return row, count


def relu_head_scores(q_row, keys):
    """q_row: [H][D] floats, keys: [n][D] floats -> n scores (double precision)."""
    dim = len(q_row[0])
    out = []
    for key in keys:
        total = 0.0
        for qh in q_row:
            dot = sum(a * b for a, b in zip(qh, key))
            total += max(dot, 0.0)
        out.append(total * dim ** -0.5)
    return out


def softmax_attend(q_vec, keys, values):
    """Single-head attention in double precision with explicit loops."""
    dim = len(q_vec)
    scores = [sum(a * b for a, b in zip(q_vec, k)) * dim ** -0.5 for k in keys]
    m = max(scores)
    w = [math.exp(s - m) for s in scores]
    z = sum(w)
    return [sum(w[t] * values[t][d] for t in range(len(keys))) / z for d in range(dim)]


# --- indexer preparation (scalar statement with emulated fp32 / bf16 rounding) ---

def f32(x):
    """Nearest fp32 (ties to even) of a Python float."""
    import struct
    return struct.unpack("<f", struct.pack("<f", x))[0]


def bf16(x):
    """Nearest bf16 (ties to even) of an fp32 value, by bit arithmetic."""
    import struct
    bits = struct.unpack("<I", struct.pack("<f", x))[0]
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def norm_rope_row(x, pos, gamma, table, eps, rotary):
    """One row: x and gamma lists of bf16 values, table a list of [cos..., sin...]
    rows (bf16 values). Every fp32 operation is one double operation on fp32
    operands (exact at these sizes) rounded by f32."""
    dim = len(x)
    ss = math.fsum(v * v for v in x)
    inv = f32(1.0 / math.sqrt(f32(f32(f32(ss) / dim) + f32(eps))))
    scaled = [bf16(f32(bf16(f32(v * inv)) * g)) for v, g in zip(x, gamma)]
    out = list(scaled)
    if rotary:
        half = rotary // 2
        row = table[pos] if 0 <= pos < len(table) else [0.0] * rotary
        for d in range(rotary):
            c = d % half
            if d < half:
                rotated = -scaled[d + half]
            else:
                rotated = scaled[d - half]
            a = bf16(f32(scaled[d] * row[c]))
            b = bf16(f32(rotated * row[half + c]))
            out[d] = bf16(f32(a + b))
    return out


def prepare_request(chunk_positions, chunk_keys, ring, ratio, state_size, k_gamma, table, eps,
                    rotary):
    """One request's compression groups and ring after a chunk.

    chunk_positions: consecutive positions of the chunk's tokens; chunk_keys:
    their raw keys; ring: {slot: key} of the ring before the chunk (slot =
    position % state_size). Walks the chunk's positions and closes a group at
    every position p with (p + 1) % ratio == 0; its members are positions
    p - ratio + 1 .. p, read from the chunk or else from the ring. Returns
    ({p: normalised pooled key}, ring after committing the chunk's last
    min(len, state_size) keys)."""
    raw = dict(zip(chunk_positions, chunk_keys))
    groups = {}
    for p in chunk_positions:
        if (p + 1) % ratio:
            continue
        members = []
        for q in range(p - ratio + 1, p + 1):
            members.append(raw[q] if q in raw else ring.get(q % state_size, [0.0] * len(k_gamma)))
        acc = [0.0] * len(k_gamma)
        for key in members:
            acc = [f32(a + v) for a, v in zip(acc, key)]
        pooled = [bf16(f32(a / ratio)) for a in acc]
        groups[p] = norm_rope_row(pooled, p - ratio + 1, k_gamma, table, eps, rotary)
    after = dict(ring)
    for p in chunk_positions[-state_size:]:
        after[p % state_size] = raw[p]
    return groups, after


def pool_rows(rows_req, rows_pos, rows_slot, qsl, ring_blocks, ring, raw, ratio, ring_size,
              raw_pos=None, ring_pos=None):
    """Per row: the mean of the group ending at its position, walking member
    positions and looking each up among the request's chunk rows (by position)
    or its ring (by position mod ring size); 0 for rows that close no valid
    group. Also the group's first position (3 columns). fp32 sums in member
    order via f32, the mean rounded to bf16."""
    out, firsts = [], []
    dim = len(raw[0])
    nreq = len(qsl) - 1
    for row, (q, end, slot) in enumerate(zip(rows_req, rows_pos, rows_slot)):
        if not (0 <= q < nreq):
            out.append([0.0] * dim)
            firsts.append([0, 0, 0])
            continue
        chunk = {}
        for r in range(qsl[q], qsl[q + 1]):
            chunk[end - (row - r)] = r        # positions run with the rows inside a chunk
        block = ring_blocks[q]
        ok = qsl[q] <= row < qsl[q + 1] and end >= ratio - 1 and slot >= 0
        if not ok:
            out.append([0.0] * dim)
            firsts.append([0, 0, 0])
            continue
        acc = [0.0] * dim
        for p in range(end - ratio + 1, end + 1):
            if p in chunk:
                key = raw[chunk[p]]
            elif p < min(chunk) and 0 <= block < len(ring):
                key = ring[block][p % ring_size]
            else:
                key = [0.0] * dim
            acc = [f32(a + v) for a, v in zip(acc, key)]
        out.append([bf16(f32(a / ratio)) for a in acc])
        first = end - ratio + 1
        if raw_pos is None:
            firsts.append([first] * 3)
        elif first in chunk:
            firsts.append(list(raw_pos[chunk[first]][:3]))
        elif 0 <= block < len(ring):
            firsts.append(list(ring_pos[block][first % ring_size][:3]))
        else:
            firsts.append([0, 0, 0])
    return out, firsts
