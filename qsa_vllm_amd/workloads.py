"""Seeded synthetic QSA workloads: paged caches, block tables and row metadata.

Builds the tensors the QSA path consumes in serving, in the layouts the
reference plugin uses:

* main KV cache: one bf16 allocation whose per-page rows hold K|V interleaved
  per (token, kv head) (``backend.py:148-153`` splits the last dim into K and
  V views ``[blocks, page, kv_heads, head_dim]``); ``token_major`` stores
  ``[blocks, page, kv_heads, 2*D]``, ``head_major`` ``[blocks, kv_heads, page, 2*D]``;
* compressed index-key cache ``[blocks, cache_page, 1, D_idx]`` with its own
  page table (one key per ``compress_ratio`` tokens, complete blocks only);
* block tables drawn from a seeded random permutation of the page pool,
  ``-1`` past each sequence's last page;
* decode rows: the last ``decode_query_len`` positions of each sequence (one
  row at position seq_len - 1 by default), visible = min((pos + 1) // ratio,
  seq_len // ratio); chunked prefill rows: positions prefix .. prefix + chunk - 1.

Activations are N(0, 1) * ``act_scale`` rounded to bf16. Everything is
generated on ``device`` from one ``torch.Generator`` seed.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import torch


@dataclass(frozen=True)
class QSAShape:
    name: str
    batch: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    compress_ratio: int
    index_heads: int
    index_dim: int
    token_topk: int
    seq_len_min: int
    seq_len_max: int
    seq_len_dist: str = "uniform"      # "uniform", "fixed" or "lognormal"
    lognormal_median: float = 65536.0
    lognormal_sigma: float = 0.5
    index_cache_page: int = 16
    pool_pages: int = 0                # 0: exactly the pages the batch needs
    act_scale: float = 1.0
    gate: bool = False
    kv_layout: str = "token_major"
    chunk: int = 0                     # > 0: chunked prefill of `chunk` new tokens per sequence
    prefix: int = 0
    decode_requests: int = 0           # with chunk > 0: the first requests decode
    decode_query_len: int = 1          # tokens per decode request (multi-token decode if > 1)
    table_tokens: int = 0              # > 0: page tables sized for this many tokens per request
    seed: int = 0

    @property
    def width(self) -> int:
        return self.token_topk + self.compress_ratio - 1


# Shapes named in the benchmark plan (one GPU's TP2 share of the serving model).
SHAPES = {
    # Eager CPU decode step: batch 4, GQA 8:1, 4096 tokens, pages from a 2048-page pool.
    "cpu_decode_4k": QSAShape(
        "cpu_decode_4k", batch=4, num_q_heads=8, num_kv_heads=1, head_dim=128, page_size=16,
        compress_ratio=16, index_heads=8, index_dim=64, token_topk=1024,
        seq_len_min=4096, seq_len_max=4096, seq_len_dist="fixed", pool_pages=2048,
        act_scale=0.5, seed=1),
    # Decode at 8k-32k context, batch 64, 16 q / 2 kv heads, top-k 2048 tokens.
    "decode_32k": QSAShape(
        "decode_32k", batch=64, num_q_heads=16, num_kv_heads=2, head_dim=128, page_size=16,
        compress_ratio=16, index_heads=32, index_dim=128, token_topk=2048,
        seq_len_min=8192, seq_len_max=32768, seed=2),
    # Chunked prefill: 4 sequences x 8192 new tokens on a 16384-token prefix.
    "prefill_8k_on_16k": QSAShape(
        "prefill_8k_on_16k", batch=4, num_q_heads=16, num_kv_heads=2, head_dim=128,
        page_size=16, compress_ratio=16, index_heads=32, index_dim=128, token_topk=2048,
        seq_len_min=24576, seq_len_max=24576, seq_len_dist="fixed", chunk=8192,
        prefix=16384, seed=3),
    # decode_32k with page tables sized for the serving max-model-len of 524288 tokens:
    # the compressed table holds 2048 pages of 16 keys, so decode scores into the
    # 32768-column width class.
    "decode_32k_serving_width": QSAShape(
        "decode_32k_serving_width", batch=64, num_q_heads=16, num_kv_heads=2, head_dim=128,
        page_size=16, compress_ratio=16, index_heads=32, index_dim=128, token_topk=2048,
        seq_len_min=8192, seq_len_max=32768, table_tokens=524288, seed=2),
    # Long-context skewed decode: batch 8, lognormal(median 64k, sigma 0.5) in [16k, 128k].
    "decode_long_skew": QSAShape(
        "decode_long_skew", batch=8, num_q_heads=16, num_kv_heads=2, head_dim=128,
        page_size=16, compress_ratio=16, index_heads=32, index_dim=128, token_topk=2048,
        seq_len_min=16384, seq_len_max=131072, seq_len_dist="lognormal", seed=4),
}


@dataclass
class QSAWorkload:
    shape: QSAShape
    device: torch.device
    seq_lens: torch.Tensor            # [requests] int32
    positions: torch.Tensor           # [rows] int64
    token_to_req: torch.Tensor        # [rows] int32
    query_start_loc: torch.Tensor     # [requests + 1] int32
    visible: torch.Tensor             # [rows] int32
    kv_cache: torch.Tensor            # physical allocation
    k_cache: torch.Tensor             # [blocks, page, kv_heads, D] view
    v_cache: torch.Tensor             # [blocks, page, kv_heads, D] view
    block_table: torch.Tensor         # [requests, pages] int32
    index_cache: torch.Tensor         # [blocks, cache_page, 1, D_idx]
    index_table: torch.Tensor         # [requests, pages] int32
    q: torch.Tensor                   # [rows, Hq, D]
    q_index: torch.Tensor             # [rows, H_idx, D_idx]
    gate: torch.Tensor | None = None
    max_seq_len: int = 0
    max_query_len: int = 1
    num_decodes: int = 0              # leading decode requests (decode_query_len rows each)
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return self.q.shape[0]

    @property
    def is_decode(self) -> bool:
        return self.shape.chunk == 0

    @property
    def num_decode_tokens(self) -> int:
        return self.num_decodes * self.shape.decode_query_len


def _seq_lens(shape: QSAShape, gen: torch.Generator) -> torch.Tensor:
    b = shape.batch
    if shape.seq_len_dist == "fixed":
        return torch.full((b,), shape.seq_len_min, dtype=torch.int64)
    if shape.seq_len_dist == "uniform":
        return torch.randint(shape.seq_len_min, shape.seq_len_max + 1, (b,), generator=gen)
    if shape.seq_len_dist == "lognormal":
        z = torch.randn(b, generator=gen, dtype=torch.float64)
        v = torch.exp(math.log(shape.lognormal_median) + shape.lognormal_sigma * z)
        return v.round().clamp(shape.seq_len_min, shape.seq_len_max).to(torch.int64)
    raise ValueError(f"unknown seq_len_dist {shape.seq_len_dist}")


def _paged_table(lengths: torch.Tensor, page: int, pool: int, gen: torch.Generator,
                 min_width: int = 0):
    """Permuted page assignment: returns (table [B, max(max_pages, min_width)]
    int32, -1 past each sequence's pages; num_blocks)."""
    pages = [(int(n) + page - 1) // page for n in lengths]
    need = sum(pages)
    num_blocks = max(need, pool, 1)
    perm = torch.randperm(num_blocks, generator=gen)
    width = max(max(pages, default=1), 1, min_width)
    table = torch.full((len(pages), width), -1, dtype=torch.int32)
    at = 0
    for i, n in enumerate(pages):
        table[i, :n] = perm[at:at + n].to(torch.int32)
        at += n
    return table, num_blocks


def _randn_bf16(shape, gen, device, scale):
    # Chunked so large caches never hold a full fp32 copy.
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
    flat = out.view(-1)
    step = 1 << 26
    for i in range(0, flat.numel(), step):
        n = min(step, flat.numel() - i)
        flat[i:i + n] = (torch.randn(n, generator=gen, device=device) * scale).to(torch.bfloat16)
    return out


def make_workload(shape: QSAShape | str, device="cpu", **overrides) -> QSAWorkload:
    """Generate a seeded workload for ``shape`` (a QSAShape or a SHAPES key)."""
    if isinstance(shape, str):
        shape = SHAPES[shape]
    if overrides:
        shape = replace(shape, **overrides)
    device = torch.device(device)
    cpu_gen = torch.Generator().manual_seed(shape.seed)
    dev_gen = torch.Generator(device=device).manual_seed(shape.seed + 1000)

    seq_lens = _seq_lens(shape, cpu_gen)
    b = shape.batch
    dql = shape.decode_query_len
    if dql < 1:
        raise ValueError("decode_query_len must be at least 1")
    # Decode requests (decode_query_len new tokens each) first, then prefill chunks.
    n_dec = min(shape.decode_requests, b) if shape.chunk else b
    q_lens = torch.tensor([dql] * n_dec + [shape.chunk] * (b - n_dec), dtype=torch.int64)
    positions = torch.cat([torch.arange(int(s) - int(n), int(s))
                           for s, n in zip(seq_lens, q_lens)])
    token_to_req = torch.arange(b, dtype=torch.int32).repeat_interleave(q_lens)
    query_start_loc = torch.cat([torch.zeros(1, dtype=torch.int64),
                                 q_lens.cumsum(0)]).to(torch.int32)
    max_query_len = int(q_lens.max())
    num_decodes = n_dec
    rows = positions.numel()
    r = shape.compress_ratio
    visible = torch.minimum((positions + 1) // r, seq_lens[token_to_req.long()] // r).to(torch.int32)

    block_table, num_blocks = _paged_table(seq_lens, shape.page_size, shape.pool_pages, cpu_gen,
                                           -(-shape.table_tokens // shape.page_size))
    index_keys = seq_lens // r
    index_table, index_blocks = _paged_table(
        index_keys, shape.index_cache_page, 0, cpu_gen,
        -(-(shape.table_tokens // r) // shape.index_cache_page))

    d, hkv = shape.head_dim, shape.num_kv_heads
    if shape.kv_layout == "token_major":
        kv = _randn_bf16((num_blocks, shape.page_size, hkv, 2 * d), dev_gen, device, shape.act_scale)
        k_cache, v_cache = kv[..., :d], kv[..., d:]
    elif shape.kv_layout == "head_major":
        kv = _randn_bf16((num_blocks, hkv, shape.page_size, 2 * d), dev_gen, device, shape.act_scale)
        k_cache, v_cache = kv.transpose(1, 2).split(d, dim=-1)
    else:
        raise ValueError(f"unknown kv_layout {shape.kv_layout}")
    index_cache = _randn_bf16((index_blocks, shape.index_cache_page, 1, shape.index_dim),
                              dev_gen, device, shape.act_scale)
    q = _randn_bf16((rows, shape.num_q_heads, d), dev_gen, device, shape.act_scale)
    q_index = _randn_bf16((rows, shape.index_heads, shape.index_dim), dev_gen, device,
                          shape.act_scale)
    gate = (_randn_bf16((rows, shape.num_q_heads, d), dev_gen, device, 1.0)
            if shape.gate else None)
    to = dict(device=device)
    return QSAWorkload(
        shape=shape, device=device,
        seq_lens=seq_lens.to(torch.int32).to(**to),
        positions=positions.to(torch.int64).to(**to),
        token_to_req=token_to_req.to(**to),
        query_start_loc=query_start_loc.to(**to),
        visible=visible.to(**to),
        kv_cache=kv, k_cache=k_cache, v_cache=v_cache,
        block_table=block_table.to(**to),
        index_cache=index_cache,
        index_table=index_table.to(**to),
        q=q, q_index=q_index, gate=gate,
        max_seq_len=int(seq_lens.max()),
        max_query_len=max_query_len,
        num_decodes=num_decodes,
    )


def fresh_queries(wl: QSAWorkload, seed: int):
    """New (q, q_index) of the workload's shapes, e.g. to rotate decode steps."""
    gen = torch.Generator(device=wl.device).manual_seed(seed)
    q = _randn_bf16(tuple(wl.q.shape), gen, wl.device, wl.shape.act_scale)
    qi = _randn_bf16(tuple(wl.q_index.shape), gen, wl.device, wl.shape.act_scale)
    return q, qi


def attention_bytes(wl: QSAWorkload, counts: torch.Tensor) -> int:
    """Algorithmic HBM bytes of one sparse-attention launch (decode rows).

    Per row: count * Hkv * 2 (K,V) * D * 2 B gathered + q and out (bf16)
    + gate if present + the W int32 indices + its count.
    """
    s = wl.shape
    gathered = int(counts.clamp_min(0).to(torch.int64).sum()) * s.num_kv_heads * 2 * s.head_dim * 2
    per_row = 2 * s.num_q_heads * s.head_dim * 2 + s.width * 4 + 4
    if wl.gate is not None:
        per_row += s.num_q_heads * s.head_dim * 2
    return gathered + wl.rows * per_row


def indexer_bytes(wl: QSAWorkload) -> int:
    """Algorithmic bytes of the decode indexer: keys + queries + logits."""
    s = wl.shape
    vis = int(wl.visible.to(torch.int64).sum())
    return vis * s.index_dim * 2 + wl.rows * s.index_heads * s.index_dim * 2 + vis * 4


def topk_bytes(wl: QSAWorkload) -> int:
    """Algorithmic bytes of the decode top-k + expansion to physical slots: the
    visible logits read, the W index columns and the count written, the
    page-table entry of every selected block and the row's position, sequence
    length and request id."""
    s = wl.shape
    vis = wl.visible.to(torch.int64)
    k = s.token_topk // s.compress_ratio
    selected = int(vis.clamp(max=k).sum())
    return int(vis.sum()) * 4 + wl.rows * ((s.width + 1) * 4 + 12) + selected * 4


def decode_step_bytes(wl: QSAWorkload, counts: torch.Tensor) -> int:
    """Algorithmic HBM bytes of one decode step: indexer + top-k + attention."""
    return indexer_bytes(wl) + topk_bytes(wl) + attention_bytes(wl, counts)


def indexer_flops(wl: QSAWorkload) -> int:
    s = wl.shape
    return 2 * s.index_heads * s.index_dim * int(wl.visible.to(torch.int64).sum())


# --- indexer preparation inputs ------------------------------------------------


@dataclass
class PrepareCase:
    """Inputs of one qsa_prepare call (ops/prepare.py:177-225) with the metadata
    its kernel reads (the upstream builder that makes it in serving is not part
    of the plugin): a ring of ``state_size`` raw keys per request, compressed
    cache pages, main K/V rows and their cache, ``k_work`` items."""

    index_qk: torch.Tensor            # [tokens, (heads + 1) * dim] view, projection row stride
    positions: torch.Tensor           # int64 [tokens]
    q_norm_weight: torch.Tensor
    k_norm_weight: torch.Tensor
    cos_sin: torch.Tensor             # bf16 [max_positions, rotary]
    eps: float
    raw: object                       # slot_mapping, block_table, query_start_loc, logical_positions
    comp: object                      # slot_mapping, k_work_metadata
    state_cache: torch.Tensor         # [blocks, state_size, dim]
    compressed_cache: torch.Tensor    # [blocks, comp_page, 1, dim]
    main_key: torch.Tensor            # [tokens, kv_heads, main_dim] view
    main_value: torch.Tensor
    main_key_cache: torch.Tensor      # [blocks, page, kv_heads, main_dim] views of main_kv
    main_value_cache: torch.Tensor
    main_slots: torch.Tensor          # int64 [tokens]
    num_index_heads: int
    index_head_dim: int
    rotary_dim: int
    compress_ratio: int
    num_groups: int                   # compression groups closed by this step
    chunk_lens: list                  # new tokens per request
    main_kv: torch.Tensor             # the K|V cache allocation [blocks, page, kv_heads, 2 * dim]
    main_block_table: torch.Tensor    # int32 [requests, pages], -1 past each sequence
    comp_table: torch.Tensor          # int32 [requests, pages] of the compressed cache
    seq_lens: torch.Tensor            # int32 [requests]: prefix + chunk
    token_to_req: torch.Tensor        # int32 [tokens]

    def call_args(self):
        """Positional and keyword arguments of qsa_prepare (both signatures)."""
        args = (self.index_qk, self.positions, self.q_norm_weight, self.k_norm_weight,
                self.cos_sin, self.eps, self.raw, self.comp, self.state_cache,
                self.compressed_cache, self.main_key, self.main_value, self.main_key_cache,
                self.main_value_cache, self.main_slots)
        kwargs = dict(num_index_heads=self.num_index_heads, index_head_dim=self.index_head_dim,
                      rotary_dim=self.rotary_dim, compress_ratio=self.compress_ratio)
        return args, kwargs

    def clone_outputs(self):
        """Copies of the tensors qsa_prepare writes (to run it twice from one state)."""
        return {"state_cache": self.state_cache.clone(),
                "compressed_cache": self.compressed_cache.clone(),
                "main_kv": self.main_kv.clone()}

    def prepare_bytes(self) -> int:
        """Algorithmic HBM bytes of one call: every byte read and written once
        (queries, raw keys of the closed groups and ring members, ring commits,
        main K/V rows, the rotary rows of the tokens, gammas)."""
        tokens = self.index_qk.shape[0]
        h, d, r = self.num_index_heads, self.index_head_dim, self.compress_ratio
        kvh, md = self.main_key.shape[1], self.main_key.shape[2]
        row = d * 2
        q = tokens * h * row * 2
        groups = self.num_groups * (r * row + row)
        ring = sum(min(c, self.state_cache.shape[1]) for c in self.chunk_lens) * row * 2
        main = int((self.main_slots >= 0).sum()) * kvh * md * 2 * 2 * 2
        rope = tokens * self.rotary_dim * 2
        return q + groups + ring + main + rope + 2 * row


def make_prepare_case(prefix_lens, chunk_lens, *, num_index_heads=32, index_head_dim=128,
                      compress_ratio=16, state_size=None, comp_page=16, main_kv_heads=2,
                      main_head_dim=128, main_page=16, rotary_dim=64, theta=1.0e7, eps=1.0e-6,
                      projection_pad=64, work_pad=3, drop_slot_every=0, history=True,
                      device="cpu", seed=0) -> PrepareCase:
    """Request q has prefix_lens[q] cached tokens and appends chunk_lens[q]
    tokens at positions prefix .. prefix + chunk - 1. index_qk, main_key and
    main_value are column slices of one projection row (as the fused QKV +
    indexer GEMM output); the ring of each request holds random raw keys of
    its earlier positions, the compressed cache random keys of its earlier
    groups and the main cache random K/V of its earlier positions, all behind
    seeded permuted page tables. drop_slot_every > 0 sets every n-th slot of
    each mapping to -1. history=False leaves the earlier compressed keys zero
    and maps only the main pages this step writes (a timing case: the
    kernel's work and slots are the same)."""
    from .ops.normalization import rotary_cache

    gen = torch.Generator(device="cpu").manual_seed(seed)
    R = compress_ratio
    S = state_size or R
    H, D = num_index_heads, index_head_dim
    prefix = [int(p) for p in prefix_lens]
    chunks = [int(c) for c in chunk_lens]
    nreq = len(chunks)
    tokens = sum(chunks)
    qsl = [0]
    for c in chunks:
        qsl.append(qsl[-1] + c)
    logical = torch.cat([torch.arange(p, p + c, dtype=torch.int64) for p, c in zip(prefix, chunks)]
                        ) if tokens else torch.zeros(0, dtype=torch.int64)
    req_of = torch.repeat_interleave(torch.arange(nreq), torch.tensor(chunks)) if tokens else \
        torch.zeros(0, dtype=torch.int64)
    max_pos = max((p + c for p, c in zip(prefix, chunks)), default=1) + 1

    # One fused projection row: [main q | main k | main v | index q heads | index k | pad].
    main_cols = main_kv_heads * main_head_dim
    idx_cols = (H + 1) * D
    cols = main_cols * 2 + idx_cols + projection_pad
    proj = (torch.randn(tokens, cols, generator=gen) * 0.5).to(torch.bfloat16)
    main_key = proj[:, :main_cols].view(tokens, main_kv_heads, main_head_dim)
    main_value = proj[:, main_cols:2 * main_cols].view(tokens, main_kv_heads, main_head_dim)
    index_qk = proj[:, 2 * main_cols:2 * main_cols + idx_cols]

    def drop(mapping):
        if drop_slot_every > 0:
            mapping[::drop_slot_every] = -1
        return mapping

    # Ring: one block per request (permuted), random earlier raw keys.
    ring_blocks = torch.randperm(nreq + 2, generator=gen)[:nreq].to(torch.int32)
    state_cache = (torch.randn(nreq + 2, S, D, generator=gen) * 0.5).to(torch.bfloat16)
    state_table = ring_blocks.view(nreq, 1).clone()
    state_slots = (ring_blocks.to(torch.int64)[req_of] * S + logical % S) if tokens else \
        torch.zeros(0, dtype=torch.int64)

    # Compressed cache pages for every group up to the end of each chunk; the
    # groups closed before the chunk hold earlier normalised keys.
    groups_total = [(p + c) // R for p, c in zip(prefix, chunks)]
    pages = [max(1, (g + comp_page - 1) // comp_page) for g in groups_total]
    comp_blocks = sum(pages) + 1
    perm = torch.randperm(comp_blocks, generator=gen).to(torch.int32)
    comp_table, at = [], 0
    for n in pages:
        comp_table.append(perm[at:at + n].tolist())
        at += n
    compressed_cache = torch.zeros(comp_blocks, comp_page, 1, D, dtype=torch.bfloat16)
    for q in range(nreq if history else 0):
        for g_ in range(prefix[q] // R):
            compressed_cache[comp_table[q][g_ // comp_page], g_ % comp_page, 0] = (
                torch.randn(D, generator=gen) * 0.5).to(torch.bfloat16)
    comp_slots = torch.full((tokens,), -1, dtype=torch.int64)
    items, closed = [], 0
    for q in range(nreq):
        chunk_start, chunk_end = prefix[q], prefix[q] + chunks[q] - 1
        n_groups = (chunk_end + 1) // R - chunk_start // R if chunks[q] else 0
        closed += max(n_groups, 0)
        for t in range(qsl[q], qsl[q + 1]):
            pos = int(logical[t])
            if (pos + 1) % R == 0:
                g = (pos + 1) // R - 1
                comp_slots[t] = comp_table[q][g // comp_page] * comp_page + g % comp_page
        if chunks[q]:
            items += [(q, w) for w in range(max(n_groups, 1))]
    perm_items = torch.randperm(len(items), generator=gen).tolist()
    items = [items[i] for i in perm_items] + [(-1, 0)] * work_pad
    k_work = torch.tensor(items, dtype=torch.int32).view(-1, 2)

    # Main cache: K|V interleaved per (token, kv head) row, permuted pages
    # holding every position of each sequence (earlier ones random); this
    # step's tokens go to their block-table slots.
    main_pages = [max(1, (p + c + main_page - 1) // main_page) for p, c in zip(prefix, chunks)]
    first_page = [0 if history else p // main_page for p in prefix]
    main_blocks = sum(n - f for n, f in zip(main_pages, first_page)) + 2
    mperm = torch.randperm(main_blocks, generator=gen).to(torch.int32)
    main_table = torch.full((nreq, max(main_pages)), -1, dtype=torch.int32)
    at = 0
    for q, n in enumerate(main_pages):
        main_table[q, first_page[q]:n] = mperm[at:at + n - first_page[q]]
        at += n - first_page[q]
    kv_shape = (main_blocks, main_page, main_kv_heads, 2 * main_head_dim)
    kv = ((torch.randn(kv_shape, generator=gen) * 0.5).to(torch.bfloat16) if history
          else torch.zeros(kv_shape, dtype=torch.bfloat16))
    main_slots = torch.zeros(tokens, dtype=torch.int64)
    for t in range(tokens):
        pos = int(logical[t])
        main_slots[t] = int(main_table[int(req_of[t]), pos // main_page]) * main_page + pos % main_page
    comp_table_t = torch.full((nreq, max(pages)), -1, dtype=torch.int32)
    for q in range(nreq):
        comp_table_t[q, :len(comp_table[q])] = torch.tensor(comp_table[q], dtype=torch.int32)

    q_w = (1.0 + 0.25 * torch.randn(D, generator=gen)).to(torch.bfloat16)
    k_w = (1.0 + 0.25 * torch.randn(D, generator=gen)).to(torch.bfloat16)
    cos_sin = rotary_cache(max_pos, rotary_dim, float(theta), "cpu") if rotary_dim else \
        torch.zeros(max_pos, 0, dtype=torch.bfloat16)

    from types import SimpleNamespace
    dev = torch.device(device)

    def to(t):
        return t.to(dev)

    # Move whole allocations so the views keep their strides.
    proj_d = to(proj)
    kv_d = to(kv)
    raw = SimpleNamespace(slot_mapping=to(drop(state_slots.clone())), block_table=to(state_table),
                          query_start_loc=to(torch.tensor(qsl, dtype=torch.int32)),
                          logical_positions=to(logical))
    comp = SimpleNamespace(slot_mapping=to(drop(comp_slots.clone())), k_work_metadata=to(k_work))
    return PrepareCase(
        index_qk=proj_d[:, 2 * main_cols:2 * main_cols + idx_cols],
        positions=to(logical.clone()), q_norm_weight=to(q_w), k_norm_weight=to(k_w),
        cos_sin=to(cos_sin.contiguous()), eps=float(eps), raw=raw, comp=comp,
        state_cache=to(state_cache), compressed_cache=to(compressed_cache),
        main_key=proj_d[:, :main_cols].view(tokens, main_kv_heads, main_head_dim),
        main_value=proj_d[:, main_cols:2 * main_cols].view(tokens, main_kv_heads, main_head_dim),
        main_key_cache=kv_d[..., :main_head_dim], main_value_cache=kv_d[..., main_head_dim:],
        main_slots=to(drop(main_slots.clone())), num_index_heads=H, index_head_dim=D,
        rotary_dim=rotary_dim, compress_ratio=R, num_groups=closed, chunk_lens=chunks, main_kv=kv_d,
        main_block_table=to(main_table), comp_table=to(comp_table_t),
        seq_lens=to(torch.tensor([p + c for p, c in zip(prefix, chunks)], dtype=torch.int32)),
        token_to_req=to(req_of.to(torch.int32)))
