"""Random-init YuLan GDN/QSA hybrid decoder at one GPU's tensor-parallel share.

The model the plugin serves (``model.py:180-226``): an embedding, decoder
layers that are either Gated DeltaNet ("linear_attention") or QSA
("full_attention") mixers, each between two gated RMSNorms and followed by a
SwiGLU MLP, a final gated norm and the LM head. Layer ``i`` is QSA when
``(i + 1) % full_attention_every == 0`` (``configuration_yulan_qsa.py:67-76``).

What runs where: the QSA layers call the path's HIP kernels through
:func:`qsa_vllm_amd.layer_step.qsa_layer_step` (prepare, select, attend); the
projections are hipBLASLt GEMMs through ``torch.nn.functional.linear``; the
gated norms, the MLP activation and the GDN mixer between its projections are
the HIP kernels of :mod:`qsa_vllm_amd.ops.hybrid_layers`.

Tensor parallelism: the weights held are one rank's share of a TP
``tp_size`` model - attention, GDN and MLP heads/intermediate divided by
``tp_size``, the indexer replicated (``attention.py:32-60``), the LM head a
vocabulary shard. The row-parallel outputs (``o_proj``, GDN ``out_proj``,
``down_proj``) are this rank's partial sums; the all-reduce that would follow
each is not part of a one-GPU step.

Per layer (``model.py:214-225``)::

    normalized, residual = input_layernorm(hidden, residual)   # residual += hidden first
    hidden = mixer(normalized)
    normalized, residual = post_attention_layernorm(hidden, residual)
    hidden = mlp(normalized)

Gated norm (``model.py:60-98``): ``n = rmsnorm(x)``;
``n * sigmoid(gate_up(silu(gate_down(n))))``. RMSNorm rounds as vLLM's kernel:
``bf16(bf16(x * rsqrt(mean(x^2) + eps)) * gamma)``; the residual add rounds to
bf16. QSA projection layout (``attention.py:25-48, 216-234``): one GEMM
``[q|gate head-interleaved, k, v, index q|k]`` with bias (zero on the index
slice), the core output gated by ``sigmoid(gate)`` inside the attention kernel.
GDN projection layout: ``in_proj_qkvz`` grouped per key head as
``[q (dk), k (dk), v (r*dv), z (r*dv)]`` and ``in_proj_ba`` as ``[b (r), a (r)]``
(the grouped layout vLLM selects with ``gqa_interleaved_layout=True``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

from .backend import QSALayerState, YuLanQSAImpl, YuLanQSAIndexer
from .graph_dispatch import capture_column_scope, check_decode_graph_batch
from .layer_step import qsa_layer_step
from .metadata import QSABatch, QSAMetadataBuilder
from .ops.hybrid_layers import (gated_norm, gdn_conv_state, gdn_gated_norm, gdn_prep,
                                gdn_recurrence, silu_mul)

__all__ = ["HybridConfig", "HybridBatch", "HybridBatchBuilder", "HybridDecoder",
           "HybridDecodeGraph", "HybridWorkload", "make_hybrid_workload",
           "make_serving_hybrid_workload", "SERVING_DECODES", "SERVING_CHUNKS", "SERVING_CHUNK"]


@dataclass(frozen=True)
class HybridConfig:
    """Model sizes (whole-model head counts; ``tp_size`` divides them)."""

    num_layers: int = 32
    full_attention_every: int = 4
    hidden_size: int = 4096
    vocab_size: int = 99072
    tp_size: int = 2
    num_heads: int = 32
    num_kv_heads: int = 4
    head_dim: int = 128
    intermediate_size: int = 11264
    linear_num_key_heads: int = 16
    linear_num_value_heads: int = 32
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    conv_kernel: int = 4
    gated_norm_rank: int = 16
    rms_norm_eps: float = 1e-6
    indexer_heads: int = 32
    indexer_head_dim: int = 128
    compress_ratio: int = 16
    token_topk: int = 2048
    rope_dim: int = 64
    rope_theta: float = 1.0e7
    page_size: int = 16
    comp_page_size: int = 16
    init_std: float = 0.02

    def layer_types(self) -> list[str]:
        return ["full_attention" if (i + 1) % self.full_attention_every == 0
                else "linear_attention" for i in range(self.num_layers)]

    @property
    def heads(self) -> int:
        return self.num_heads // self.tp_size

    @property
    def kv_heads(self) -> int:
        return self.num_kv_heads // self.tp_size

    @property
    def key_heads(self) -> int:
        return self.linear_num_key_heads // self.tp_size

    @property
    def value_heads(self) -> int:
        return self.linear_num_value_heads // self.tp_size

    @property
    def intermediate(self) -> int:
        return self.intermediate_size // self.tp_size

    @property
    def vocab_shard(self) -> int:
        return self.vocab_size // self.tp_size

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_heads * self.linear_key_head_dim + self.value_heads * self.linear_value_head_dim

    @property
    def output_width(self) -> int:
        return self.token_topk + self.compress_ratio - 1


class _Init:
    """Seeded N(0, std) bf16 tensors generated on the device."""

    def __init__(self, device, seed: int, std: float):
        self.device = torch.device(device)
        self.gen = torch.Generator(device=self.device).manual_seed(seed)
        self.std = std

    def normal(self, *shape, std=None, dtype=torch.bfloat16):
        out = torch.empty(shape, dtype=dtype, device=self.device)
        flat = out.view(-1)
        step = 1 << 26
        for i in range(0, flat.numel(), step):
            n = min(step, flat.numel() - i)
            flat[i:i + n] = torch.randn(n, generator=self.gen, device=self.device) * (
                self.std if std is None else std)
        return out

    def uniform(self, *shape, low=0.0, high=1.0):
        return torch.rand(shape, generator=self.gen, device=self.device) * (high - low) + low


class GatedNorm:
    """``YuLanGatedNorm`` (``model.py:60-98``) with vLLM's fused residual add:
    ``norm(x, residual)`` adds ``x`` into ``residual`` in place."""

    def __init__(self, cfg: HybridConfig, init: _Init):
        h, r = cfg.hidden_size, cfg.gated_norm_rank
        self.eps = cfg.rms_norm_eps
        self.weight = torch.ones(h, dtype=torch.bfloat16, device=init.device)
        self.gate_down = init.normal(r, h)
        self.gate_up = init.normal(h, r)
        self.gate_up_bias = init.normal(h)

    def __call__(self, x, residual=None):
        gated, res = gated_norm(x, residual, self.weight, self.gate_down, self.gate_up,
                                self.gate_up_bias, self.eps)
        return gated if residual is None else (gated, res)


class SwiGLU:
    """``Qwen2MoeMLP`` with ``hidden_act="silu"``: ``down(silu(gate) * up)``."""

    def __init__(self, cfg: HybridConfig, init: _Init):
        self.gate_up_proj = init.normal(2 * cfg.intermediate, cfg.hidden_size)
        self.down_proj = init.normal(cfg.hidden_size, cfg.intermediate)

    def __call__(self, x):
        return F.linear(silu_mul(F.linear(x, self.gate_up_proj)), self.down_proj)


class QSAAttention:
    """``YuLanQSAAttention.forward`` + ``_run_qsa`` (``attention.py:145-234``)."""

    def __init__(self, cfg: HybridConfig, init: _Init, kv_cache, ring_cache, comp_cache,
                 max_tokens: int, max_position: int):
        d = cfg.head_dim
        self.heads, self.kv_heads, self.head_dim = cfg.heads, cfg.kv_heads, d
        self.q_size = self.heads * d * 2
        self.kv_size = self.kv_heads * d
        self.index_size = (cfg.indexer_heads + 1) * cfg.indexer_head_dim
        rows = self.q_size + 2 * self.kv_size + self.index_size
        self.qkv_weight = init.normal(rows, cfg.hidden_size)
        self.qkv_bias = init.normal(rows)
        self.qkv_bias[-self.index_size:] = 0
        self.o_proj = init.normal(cfg.hidden_size, self.heads * d)
        self.indexer = YuLanQSAIndexer(cfg.indexer_heads, cfg.indexer_head_dim, cfg.compress_ratio,
                                       cfg.token_topk, cfg.rope_dim, cfg.rope_theta,
                                       cfg.rms_norm_eps, max_position, ring_cache, comp_cache)
        self.layer = QSALayerState(kv_cache, d, max_tokens, cfg.output_width)
        self.impl = YuLanQSAImpl(self.heads, self.kv_heads, d)

    def split(self, qkv):
        """(query, gate, key, value, index_qk) views of the projection output."""
        t, d = qkv.shape[0], self.head_dim
        q, k, v, index_qk = qkv.split((self.q_size, self.kv_size, self.kv_size, self.index_size),
                                      dim=-1)
        qg = q.view(t, self.heads, 2 * d)
        return (qg[..., :d], qg[..., d:], k.view(t, self.kv_heads, d),
                v.view(t, self.kv_heads, d), index_qk)

    def __call__(self, x, batch: "HybridBatch"):
        t = x.shape[0]
        qkv = F.linear(x, self.qkv_weight, self.qkv_bias)
        query, gate, key, value, index_qk = self.split(qkv)
        core = torch.empty(t, self.heads, self.head_dim, dtype=torch.bfloat16, device=x.device)
        qsa_layer_step(self.indexer, self.impl, self.layer, batch.qsa, index_qk, key, value, query,
                       core, gate)
        return F.linear(core.view(t, -1), self.o_proj)


class GatedDeltaNet:
    """The GDN mixer (``QwenGatedDeltaNetAttention``) with its recurrent
    state (fp32 ``[slots, value_heads, dk, dv]``) and conv state (bf16
    ``[slots, K-1, conv_dim]``)."""

    def __init__(self, cfg: HybridConfig, init: _Init, num_slots: int, state_std: float):
        hk, hv = cfg.key_heads, cfg.value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        self.hk, self.hv, self.dk, self.dv, self.r = hk, hv, dk, dv, hv // hk
        self.eps = cfg.rms_norm_eps
        self.n_qkvz = hk * (2 * dk + 2 * self.r * dv)
        qkvz_w = init.normal(self.n_qkvz, cfg.hidden_size)
        ba_w = init.normal(2 * hv, cfg.hidden_size)
        # One projection GEMM per call: in_proj_qkvz and in_proj_ba are row
        # blocks of one weight, their outputs column blocks of one product
        # (the GDN kernels take row strides, which must be multiples of 8
        # elements: zero rows pad the weight to that, for any head count).
        pad = -(self.n_qkvz + 2 * hv) % 8
        self.in_proj = torch.cat([qkvz_w, ba_w, qkvz_w.new_zeros(pad, cfg.hidden_size)])
        del qkvz_w, ba_w
        if self.in_proj.shape[0] % 8:
            raise ValueError("GDN projection rows must pad to a multiple of 8")
        self.in_proj_qkvz = self.in_proj[:self.n_qkvz]
        self.in_proj_ba = self.in_proj[self.n_qkvz:self.n_qkvz + 2 * hv]
        self.conv_weight = init.normal(cfg.conv_dim, cfg.conv_kernel, std=0.5)
        self.A_log = init.uniform(hv, low=1.0, high=16.0).log()
        self.dt_bias = torch.ones(hv, dtype=torch.float32, device=init.device)
        self.norm_weight = torch.ones(dv, dtype=torch.bfloat16, device=init.device)
        self.out_proj = init.normal(cfg.hidden_size, hv * dv)
        self.conv_state = init.normal(num_slots, cfg.conv_kernel - 1, cfg.conv_dim, std=1.0)
        self.ssm_state = init.normal(num_slots, hv, dk, dv, std=state_std, dtype=torch.float32)

    def __call__(self, x, batch: "HybridBatch"):
        t = x.shape[0]
        proj = F.linear(x, self.in_proj)
        qkvz, ba = proj[:, :self.n_qkvz], proj[:, self.n_qkvz:self.n_qkvz + 2 * self.hv]
        q, k, v, g, beta = gdn_prep(qkvz, ba, self.conv_weight, self.conv_state,
                                    batch.query_start_loc, batch.token_to_seq, batch.state_slots,
                                    self.A_log, self.dt_bias, self.hk, self.hv)
        gdn_conv_state(qkvz, self.conv_state, batch.query_start_loc, batch.state_slots, self.hk,
                       self.hv)
        o = gdn_recurrence(q, k, v, g, beta, self.ssm_state, batch.query_start_loc,
                           batch.state_slots, self.hk, self.hv,
                           max_query_len=batch.qsa.main.max_query_len)
        y = gdn_gated_norm(o, qkvz, self.norm_weight, self.eps, self.hk, self.hv)
        return F.linear(y.view(t, -1), self.out_proj)


class DecoderLayer:
    """``YuLanQSADecoderLayer`` (``model.py:180-225``)."""

    def __init__(self, kind: str, mixer, cfg: HybridConfig, init: _Init):
        self.kind = kind
        self.mixer = mixer
        self.input_layernorm = GatedNorm(cfg, init)
        self.post_attention_layernorm = GatedNorm(cfg, init)
        self.mlp = SwiGLU(cfg, init)

    def __call__(self, hidden, residual, batch):
        if residual is None:
            residual = hidden
            normalized = self.input_layernorm(hidden)
        else:
            normalized, residual = self.input_layernorm(hidden, residual)
        hidden = self.mixer(normalized, batch)
        normalized, residual = self.post_attention_layernorm(hidden, residual)
        return self.mlp(normalized), residual


@dataclass
class HybridBatch:
    """One step's inputs: token ids, the QSA metadata (shared by every QSA
    layer; its request ranges are the GDN sequences) and the GDN state slots."""

    token_ids: torch.Tensor            # int64 [tokens]
    qsa: QSABatch
    num_decode_tokens: int             # leading one-token requests
    state_slots: torch.Tensor          # int64 [requests]
    logits_rows: torch.Tensor          # int64 [requests]: each request's last token

    @property
    def num_tokens(self) -> int:
        return self.qsa.num_tokens

    @property
    def query_start_loc(self) -> torch.Tensor:
        return self.qsa.raw.query_start_loc

    @property
    def token_to_seq(self) -> torch.Tensor:
        return self.qsa.token_to_req


class HybridBatchBuilder:
    """Builds :class:`HybridBatch` from scheduler-level inputs (tokens already
    computed and scheduled per request, decode requests first). Every tensor
    of a batch is a view of a persistent device buffer refreshed by ``build``,
    so a graph captured on one batch reads the next batch's values on replay."""

    def __init__(self, cfg: HybridConfig, *, max_requests: int, max_tokens: int,
                 main_table_width: int, comp_table_width: int, device):
        self.cfg = cfg
        self.device = torch.device(device)
        self.qsa = QSAMetadataBuilder(
            compress_ratio=cfg.compress_ratio, main_page_size=cfg.page_size,
            comp_page_size=cfg.comp_page_size, ring_size=cfg.compress_ratio,
            max_num_requests=max_requests, max_num_tokens=max_tokens,
            main_table_width=main_table_width, comp_table_width=comp_table_width, device=device)
        self.token_ids = torch.zeros(max_tokens, dtype=torch.int64, device=self.device)
        self.state_slots = torch.full((max_requests,), -1, dtype=torch.int64, device=self.device)
        self.logits_rows = torch.zeros(max_requests, dtype=torch.int64, device=self.device)

    def _fill(self, dst, a):
        t = torch.as_tensor(np.ascontiguousarray(a), dtype=dst.dtype)
        if self.device.type == "cuda":
            t = t.pin_memory()
        dst[:t.numel()].copy_(t, non_blocking=True)
        return dst[:t.numel()]

    def build(self, computed, scheduled, token_ids, main_table, comp_table, ring_blocks,
              state_slots) -> HybridBatch:
        qsa = self.qsa.build(computed, scheduled, main_table, comp_table, ring_blocks)
        sched = np.asarray(scheduled, dtype=np.int64)
        return HybridBatch(token_ids=self._fill(self.token_ids, token_ids), qsa=qsa,
                           num_decode_tokens=qsa.compressed.num_decodes,
                           state_slots=self._fill(self.state_slots, np.asarray(state_slots)),
                           logits_rows=self._fill(self.logits_rows, np.cumsum(sched) - 1))


class HybridDecoder:
    """``YuLanQSAModel`` + LM head shard (``model.py:228-290``)."""

    def __init__(self, cfg: HybridConfig, *, num_blocks: int, comp_blocks: int, ring_blocks: int,
                 state_slots: int, max_tokens: int, max_position: int, device, seed: int = 0,
                 cache_std: float = 1.0, state_std: float = 0.02):
        init = _Init(device, seed, cfg.init_std)
        self.cfg = cfg
        self.embed_tokens = init.normal(cfg.vocab_size, cfg.hidden_size)
        self.layers = []
        d, dx = cfg.head_dim, cfg.indexer_head_dim
        for kind in cfg.layer_types():
            if kind == "full_attention":
                kv = init.normal(num_blocks, cfg.page_size, cfg.kv_heads, 2 * d, std=cache_std)
                ring = init.normal(ring_blocks, cfg.compress_ratio, dx, std=cache_std)
                comp = init.normal(comp_blocks, cfg.comp_page_size, 1, dx, std=cache_std)
                mixer = QSAAttention(cfg, init, kv.permute(0, 2, 1, 3), ring, comp, max_tokens,
                                     max_position)
            else:
                mixer = GatedDeltaNet(cfg, init, state_slots, state_std)
            self.layers.append(DecoderLayer(kind, mixer, cfg, init))
        self.norm = GatedNorm(cfg, init)
        self.lm_head = init.normal(cfg.vocab_shard, cfg.hidden_size)

    def embed(self, token_ids):
        return F.embedding(token_ids, self.embed_tokens)

    def logits(self, hidden, residual, batch):
        normalized, _ = self.norm(hidden, residual)
        return F.linear(normalized[batch.logits_rows], self.lm_head).float()

    def forward(self, batch: HybridBatch) -> torch.Tensor:
        """One step: fp32 logits [requests, vocab shard] of each request's last token."""
        hidden, residual = self.embed(batch.token_ids), None
        for layer in self.layers:
            hidden, residual = layer(hidden, residual, batch)
        return self.logits(hidden, residual, batch)


class HybridDecodeGraph:
    """``HybridDecoder.forward`` captured for a uniform decode batch (one token
    per request) of one size, replayed after the builder refreshes its
    buffers. ``columns`` pins the decode logits-width class during capture (0:
    the compressed page table's capacity). Capture runs the step once as a
    warm-up, which advances the caches and states like any step."""

    def __init__(self, model: "HybridDecoder", batch: HybridBatch, columns: int = 0):
        if batch.qsa.main.max_query_len != 1:
            raise ValueError("graphs are captured for uniform decode batches only")
        self.num_tokens = batch.num_tokens
        self.columns = columns
        self.compress_ratio = model.cfg.compress_ratio
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with capture_column_scope(columns), torch.cuda.stream(side):
            model.forward(batch)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with capture_column_scope(columns), torch.cuda.graph(self.graph):
            self.logits = model.forward(batch)

    def replay(self, batch: HybridBatch | None = None) -> torch.Tensor:
        """Replay on the builder's current buffers; returns the logits buffer."""
        if batch is not None:
            check_decode_graph_batch(batch.qsa, self.num_tokens, self.columns,
                                     self.compress_ratio)
        self.graph.replay()
        return self.logits


@dataclass
class HybridWorkload:
    """A seeded mixed batch: requests, page tables, GDN slots and the model."""

    cfg: HybridConfig
    model: HybridDecoder
    builder: HybridBatchBuilder
    computed: list
    scheduled: list
    token_ids: np.ndarray
    main_table: torch.Tensor
    comp_table: torch.Tensor
    ring_blocks: torch.Tensor
    state_slots: np.ndarray
    extra: dict = field(default_factory=dict)

    @property
    def num_tokens(self) -> int:
        return int(sum(self.scheduled))

    def build(self) -> HybridBatch:
        return self.builder.build(self.computed, self.scheduled, self.token_ids, self.main_table,
                                  self.comp_table, self.ring_blocks, self.state_slots)

    def build_decode(self) -> HybridBatch:
        """A uniform decode batch of the workload's decode requests (the
        leading one-token requests), one more token each."""
        n = 0
        while n < len(self.scheduled) and self.scheduled[n] == 1:
            n += 1
        if n == 0:
            raise ValueError("the workload has no decode requests")
        return self.builder.build(self.computed[:n], [1] * n, self.token_ids[:n],
                                  self.main_table[:n], self.comp_table[:n], self.ring_blocks[:n],
                                  self.state_slots[:n])

    def layer_states(self) -> list[torch.Tensor]:
        """Every tensor a step writes (caches and recurrent states), for tests
        that restore a starting point."""
        out = []
        for layer in self.model.layers:
            mx = layer.mixer
            if layer.kind == "full_attention":
                out += [mx.layer.kv_cache, mx.indexer.raw_key_cache, mx.indexer.compressed_key_cache]
            else:
                out += [mx.conv_state, mx.ssm_state]
        return out


def make_hybrid_workload(cfg: HybridConfig, *, decode_lens, chunk_prefixes, chunk: int, device,
                         seed: int = 0, cache_std: float = 1.0, state_std: float = 0.02,
                         spare_pages: int = 3) -> HybridWorkload:
    """Decode requests with ``decode_lens`` tokens already computed (one new
    token each), then prefill chunks of ``chunk`` tokens on ``chunk_prefixes``.
    Pages come from a seeded permutation of the pool."""
    gen = torch.Generator().manual_seed(seed)
    computed = [int(n) for n in decode_lens] + [int(p) for p in chunk_prefixes]
    scheduled = [1] * len(decode_lens) + [int(chunk)] * len(chunk_prefixes)
    totals = [c + s for c, s in zip(computed, scheduled)]
    nreq = len(totals)
    page, cpage, R = cfg.page_size, cfg.comp_page_size, cfg.compress_ratio
    main_pages = [-(-n // page) for n in totals]
    comp_pages = [max(1, -(-(n // R) // cpage)) for n in totals]

    def table(pages, extra):
        pool = sum(pages) + extra
        perm = torch.randperm(pool, generator=gen).to(torch.int32)
        t = torch.full((nreq, max(pages)), -1, dtype=torch.int32)
        at = 0
        for i, n in enumerate(pages):
            t[i, :n] = perm[at:at + n]
            at += n
        return t, pool

    main_table, num_blocks = table(main_pages, spare_pages)
    comp_table, comp_blocks = table(comp_pages, spare_pages)
    ring_blocks = torch.randperm(nreq + spare_pages, generator=gen)[:nreq].to(torch.int32)
    state_slots = torch.randperm(nreq + spare_pages, generator=gen)[:nreq].numpy()
    tokens = sum(scheduled)
    token_ids = torch.randint(0, cfg.vocab_size, (tokens,), generator=gen).numpy()
    max_position = -(-max(totals) // 4096) * 4096
    model = HybridDecoder(cfg, num_blocks=num_blocks, comp_blocks=comp_blocks,
                          ring_blocks=nreq + spare_pages, state_slots=nreq + spare_pages,
                          max_tokens=tokens, max_position=max_position, device=device, seed=seed,
                          cache_std=cache_std, state_std=state_std)
    builder = HybridBatchBuilder(cfg, max_requests=nreq, max_tokens=tokens,
                                 main_table_width=main_table.shape[1],
                                 comp_table_width=comp_table.shape[1], device=device)
    dev = torch.device(device)
    return HybridWorkload(cfg=cfg, model=model, builder=builder, computed=computed,
                          scheduled=scheduled, token_ids=token_ids, main_table=main_table.to(dev),
                          comp_table=comp_table.to(dev), ring_blocks=ring_blocks,
                          state_slots=state_slots)


# The serving batch of the hybrid step: 112 decode requests at contexts
# U[4096, 32768], then 16 prefill chunks of 512 tokens on prefixes 512 * U{0..31}.
SERVING_DECODES, SERVING_CHUNKS, SERVING_CHUNK = 112, 16, 512


def make_serving_hybrid_workload(device, seed: int = 11,
                                 cfg: HybridConfig | None = None) -> HybridWorkload:
    """The full-size model (32 layers, hidden 4096, TP2 share) on the mixed
    continuous batch of 112 decode requests and 16 prefill chunks (8304 tokens)."""
    rng = np.random.default_rng(seed)
    decode_lens = rng.integers(4096, 32768, SERVING_DECODES, endpoint=True).tolist()
    prefixes = (SERVING_CHUNK * rng.integers(0, 32, SERVING_CHUNKS)).tolist()
    return make_hybrid_workload(cfg or HybridConfig(), decode_lens=decode_lens,
                                chunk_prefixes=prefixes, chunk=SERVING_CHUNK, device=device,
                                seed=seed)
