"""Batch metadata of the QSA path, built from scheduler-level inputs.

In serving, vLLM's QSA cache builder (``vllm.models.qwen4_exp.common.qsa_cache``,
not part of the plugin) produces the compressed-key and raw-ring metadata and
the main attention gets its page table and write slots
(``metadata.py:29-62``). :class:`QSAMetadataBuilder` produces every field the
path reads from what a scheduler knows about a batch: per request, the tokens
already computed and the tokens scheduled now, plus the page tables of the
main cache, the compressed-key cache and the raw-key ring.

All tensors live in persistent device buffers sized at construction, so a
HIP graph captured over the path reads each new batch's metadata on replay;
``build`` refreshes them on the current stream and returns views of the
batch's length. Requests are taken in the given order: the leading requests
that schedule exactly ``decode_query_len`` tokens (1, or more for multi-token
decode such as speculative verification) are the decode part (the plugin's
decode-first row order, request i owning rows ``[i * dql, (i + 1) * dql)``,
``ops/indexer.py:227-279``), the rest are prefill.

Fields (per token t of request q at position p, ratio R):

* position ``p``, ``token_to_req[t] = q``, ``seq_lens[q]`` = computed + scheduled;
* main slot ``main_table[q, p // page] * page + p % page``;
* ring slot ``ring_block[q] * ring + p % ring``;
* compressed slot of the group that ends at ``p`` (``(p + 1) % R == 0``):
  ``comp_table[q, g // cpage] * cpage + g % cpage`` with ``g = (p + 1) / R - 1``, else -1;
* ``visible_blocks[t] = min((p + 1) // R, seq_len // R)`` (``ops/indexer.py:363-369``);
* ``k_work``: ``max(1, groups closed by the chunk)`` items ``(q, w)`` per request
  (item 0 also commits the ring), padded with ``(-1, 0)`` to the buffer's capacity
  (``ops/prepare.py:120-174``).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .backend import QSACompressedMetadata, QSARawMetadata, YuLanQSAMetadata


@dataclass
class QSABatch:
    """One batch's metadata (views of the builder's buffers)."""

    num_tokens: int
    num_requests: int
    positions: torch.Tensor          # int64 [tokens]
    token_to_req: torch.Tensor       # int32 [tokens]
    main: YuLanQSAMetadata
    raw: QSARawMetadata
    compressed: QSACompressedMetadata


class QSAMetadataBuilder:
    def __init__(self, *, compress_ratio: int, main_page_size: int, comp_page_size: int,
                 ring_size: int, max_num_requests: int, max_num_tokens: int,
                 main_table_width: int, comp_table_width: int, device):
        self.R = compress_ratio
        self.main_page = main_page_size
        self.comp_page = comp_page_size
        self.ring = ring_size
        self.max_requests = max_num_requests
        self.max_tokens = max_num_tokens
        dev = torch.device(device)
        self.device = dev

        def buf(shape, dtype, fill=0):
            return torch.full(shape, fill, dtype=dtype, device=dev)

        self.query_start_loc = buf((max_num_requests + 1,), torch.int32)
        self.seq_lens = buf((max_num_requests,), torch.int32)
        self.positions = buf((max_num_tokens,), torch.int64)
        self.token_to_req = buf((max_num_tokens,), torch.int32)
        self.visible = buf((max_num_tokens,), torch.int32)
        self.main_slots = buf((max_num_tokens,), torch.int64, -1)
        self.ring_slots = buf((max_num_tokens,), torch.int64, -1)
        self.comp_slots = buf((max_num_tokens,), torch.int64, -1)
        self.main_table = buf((max_num_requests, main_table_width), torch.int32, -1)
        self.comp_table = buf((max_num_requests, comp_table_width), torch.int32, -1)
        self.ring_table = buf((max_num_requests, 1), torch.int32, -1)
        # Every request has at least one item; a chunk of n tokens closes at
        # most n // R + 1 groups.
        self.k_work_capacity = max_num_requests + max_num_tokens // compress_ratio + 1
        self.k_work = buf((self.k_work_capacity, 2), torch.int32)

    def build(self, num_computed_tokens, num_scheduled_tokens, main_block_table: torch.Tensor,
              comp_block_table: torch.Tensor, ring_blocks, *,
              decode_query_len: int = 1) -> QSABatch:
        if decode_query_len < 1:
            raise ValueError(f"decode_query_len must be at least 1, got {decode_query_len}")
        computed = np.asarray(num_computed_tokens, dtype=np.int64)
        scheduled = np.asarray(num_scheduled_tokens, dtype=np.int64)
        nreq = int(scheduled.size)
        if nreq > self.max_requests or scheduled.sum() > self.max_tokens:
            raise ValueError("batch exceeds the builder's request or token capacity")
        if (scheduled <= 0).any() or (computed < 0).any():
            raise ValueError("every request must schedule at least one token")
        tokens = int(scheduled.sum())
        R = self.R
        qsl = np.zeros(nreq + 1, dtype=np.int32)
        np.cumsum(scheduled, out=qsl[1:])
        req = np.repeat(np.arange(nreq, dtype=np.int32), scheduled)
        pos = (np.repeat(computed, scheduled)
               + np.arange(tokens, dtype=np.int64) - np.repeat(qsl[:-1].astype(np.int64), scheduled))
        seq = (computed + scheduled).astype(np.int32)
        visible = np.minimum((pos + 1) // R, seq[req] // R).astype(np.int32)
        first = computed // R
        groups = (computed + scheduled) // R - first
        items = [(q, w) for q in range(nreq) for w in range(max(int(groups[q]), 1))]
        k_work = np.zeros((self.k_work_capacity, 2), dtype=np.int32)
        k_work[:, 0] = -1
        k_work[:len(items)] = np.asarray(items, dtype=np.int32).reshape(-1, 2)

        dev = self.device
        host = {
            "query_start_loc": torch.from_numpy(qsl),
            "seq_lens": torch.from_numpy(seq),
            "positions": torch.from_numpy(pos),
            "token_to_req": torch.from_numpy(req),
            "visible": torch.from_numpy(visible),
            "k_work": torch.from_numpy(k_work),
        }
        for name, t in host.items():
            dst = getattr(self, name)
            dst[:t.shape[0]].copy_(t.pin_memory() if dev.type == "cuda" else t, non_blocking=True)
        for dst, src in ((self.main_table, main_block_table), (self.comp_table, comp_block_table)):
            if src.shape[0] < nreq or src.shape[1] > dst.shape[1]:
                raise ValueError("page table has fewer rows than requests or more columns than "
                                 "the builder holds")
            dst[:nreq].fill_(-1)
            dst[:nreq, :src.shape[1]].copy_(src[:nreq])
        self.ring_table[:nreq, 0].copy_(torch.as_tensor(ring_blocks, dtype=torch.int32)[:nreq])

        def lookup(table, index):
            # table[q, index], -1 where index is past the table's width
            inside = index < table.shape[1]
            entry = table[:nreq][q, torch.where(inside, index, torch.zeros_like(index))].long()
            return torch.where(inside, entry, torch.full_like(entry, -1))

        # Slot mappings on the device, from the page tables already there.
        p = self.positions[:tokens]
        q = self.token_to_req[:tokens].long()
        main_page = lookup(self.main_table, p // self.main_page)
        self.main_slots[:tokens].copy_(torch.where(main_page >= 0,
                                                   main_page * self.main_page + p % self.main_page,
                                                   torch.full_like(p, -1)))
        ring_block = self.ring_table[:nreq, 0][q].long()
        self.ring_slots[:tokens].copy_(torch.where(ring_block >= 0, ring_block * self.ring + p % self.ring,
                                                   torch.full_like(p, -1)))
        g = (p + 1) // R - 1
        closes = (p + 1) % R == 0
        gi = torch.where(closes, g, torch.zeros_like(g))
        comp_page = lookup(self.comp_table, gi // self.comp_page)
        self.comp_slots[:tokens].copy_(torch.where(
            closes & (comp_page >= 0), comp_page * self.comp_page + gi % self.comp_page,
            torch.full_like(p, -1)))

        decode_requests = 0
        while decode_requests < nreq and scheduled[decode_requests] == decode_query_len:
            decode_requests += 1
        max_query_len = int(scheduled.max())
        max_seq_len = int(seq.max())
        main = YuLanQSAMetadata(num_actual_tokens=tokens, max_query_len=max_query_len,
                                block_table=self.main_table[:nreq],
                                slot_mapping=self.main_slots[:tokens])
        raw = QSARawMetadata(slot_mapping=self.ring_slots[:tokens],
                             block_table=self.ring_table[:nreq],
                             query_start_loc=self.query_start_loc[:nreq + 1],
                             logical_positions=self.positions[:tokens])
        compressed = QSACompressedMetadata(
            block_table=self.comp_table[:nreq], token_to_req=self.token_to_req[:tokens],
            logical_positions=self.positions[:tokens], seq_lens=self.seq_lens[:nreq],
            query_start_loc=self.query_start_loc[:nreq + 1], max_query_len=max_query_len,
            max_seq_len=max_seq_len, num_decodes=decode_requests,
            num_decode_tokens=decode_requests * decode_query_len,
            decode_query_len=decode_query_len,
            visible_blocks=self.visible[:tokens], slot_mapping=self.comp_slots[:tokens],
            k_work_metadata=self.k_work)
        return QSABatch(num_tokens=tokens, num_requests=nreq, positions=self.positions[:tokens],
                        token_to_req=self.token_to_req[:tokens], main=main, raw=raw,
                        compressed=compressed)
