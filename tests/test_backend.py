"""The attention-side glue (``qsa_vllm_amd.backend``): cache views, the layer
call order and the decode / prefill / mixed flags, against the oracle."""

import pytest
import torch

import oracle
from qsa_vllm_amd.workloads import make_workload

DEV = "cuda:0"
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _backend():
    from qsa_vllm_amd import backend  # loads libqsa_hip.so (no GPU needed to load it)
    return backend


@pytest.mark.parametrize("heads", [1, 2])
@pytest.mark.parametrize("layout", ["BLNHC", "BLHNC"])
def test_main_kv_views_address_the_bound_cache(heads, layout):
    """backend.py:148-153: the logical [blocks, heads, page, 2D] view the cache is
    bound as, whatever the physical layout, gives K/V [blocks, page, heads, D]."""
    backend = _backend()
    blocks, page, d = 3, 16, 8
    g = torch.Generator().manual_seed(heads)
    if layout == "BLNHC":   # physical [blocks, page, heads, 2D]
        phys = torch.randn(blocks, page, heads, 2 * d, generator=g)
        bound = phys.permute(0, 2, 1, 3)
        want_k, want_v = phys[..., :d], phys[..., d:]
    else:                   # physical [blocks, heads, page, 2D]
        phys = torch.randn(blocks, heads, page, 2 * d, generator=g)
        bound = phys
        want_k, want_v = phys.transpose(1, 2)[..., :d], phys.transpose(1, 2)[..., d:]
    k, v = backend.main_kv_views(bound, d)
    assert k.shape == (blocks, page, heads, d) and v.shape == k.shape
    assert torch.equal(k, want_k) and torch.equal(v, want_v)
    assert k.data_ptr() == phys.data_ptr() and v.data_ptr() == phys.data_ptr() + d * 4
    assert k.stride(3) == 1
    if heads == 1:
        assert k.stride(2) == d          # canonical stride of the singleton head dim


def test_canonical_strides_keep_addresses():
    backend = _backend()
    base = torch.arange(2 * 1 * 5 * 1 * 4, dtype=torch.float32).view(2, 5, 4)
    t = base.unsqueeze(1).unsqueeze(3)        # [2, 1, 5, 1, 4]
    weird = t.as_strided(t.shape, (20, 777, 4, 999, 1))
    c = backend.canonicalize_singleton_dim_strides(weird)
    assert c.stride() == (20, 20, 4, 4, 1)
    assert torch.equal(c, t)


def _check_attn(got, want, what):
    err = (got.float().cpu() - want).abs()
    print(f"[backend] {what}: max_abs={err.max().item():.3e} mean_abs={err.mean().item():.3e}",
          flush=True)
    assert err.max().item() <= MAX_ABS and err.mean().item() <= MEAN_ABS, what


def _compressed_meta(backend, wl):
    return backend.QSACompressedMetadata(
        block_table=wl.index_table, token_to_req=wl.token_to_req,
        logical_positions=wl.positions, seq_lens=wl.seq_lens,
        query_start_loc=wl.query_start_loc, max_query_len=wl.max_query_len,
        max_seq_len=wl.max_seq_len, num_decodes=wl.num_decodes,
        num_decode_tokens=wl.num_decode_tokens, decode_query_len=wl.shape.decode_query_len,
        visible_blocks=wl.visible)


def _gpu_logits(wl):
    """The fp32 logits the HIP scorers produce for the workload's rows
    (decode rows, then prefill rows), each part at its own width."""
    from qsa_vllm_amd.graph_dispatch import decode_logits_columns, prefill_logits_width
    s = wl.shape
    nd = wl.num_decode_tokens
    cap = wl.index_table.shape[1] * wl.index_cache.shape[1]
    parts = []
    if nd:
        cols = decode_logits_columns(wl.max_seq_len, s.compress_ratio, cap)
        lg = torch.full((nd, cols), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_decode(wl.q_index[:nd], wl.index_cache,
                                                   wl.index_table[:wl.num_decodes],
                                                   wl.visible[:nd], lg,
                                                   wl.shape.decode_query_len)
        parts.append(lg.cpu())
    if nd < wl.rows:
        width = prefill_logits_width(wl.max_seq_len, s.compress_ratio, cap)
        n = wl.rows - nd
        lg = torch.full((n, width), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_prefill(
            wl.q_index[nd:], wl.index_cache, wl.index_table[wl.num_decodes:],
            wl.query_start_loc[wl.num_decodes:], wl.visible[nd:], lg, 0, n, wl.max_query_len)
        parts.append(lg.cpu())
    return parts


def _run_layer(wl, pad_rows=3):
    backend = _backend()
    s = wl.shape
    rows = wl.rows
    layer = backend.QSALayerState(wl.kv_cache.permute(0, 2, 1, 3)
                                  if s.kv_layout == "token_major" else wl.kv_cache,
                                  s.head_dim, rows + pad_rows, s.width)
    impl = backend.YuLanQSAImpl(s.num_q_heads, s.num_kv_heads, s.head_dim)
    main = backend.YuLanQSAMetadata(num_actual_tokens=rows, max_query_len=wl.max_query_len,
                                    block_table=wl.block_table,
                                    slot_mapping=torch.zeros(rows, dtype=torch.int64, device=DEV))
    output = torch.full((rows + pad_rows, s.num_q_heads, s.head_dim), float("nan"),
                        dtype=torch.bfloat16, device=DEV)
    backend.run_qsa(layer, impl, wl.q_index, wl.index_cache, wl.q, wl.gate, output, main,
                    _compressed_meta(backend, wl), s.token_topk, s.compress_ratio,
                    wl.token_to_req)
    torch.cuda.synchronize()
    return layer, output


def _expected_selection(wl, physical):
    s = wl.shape
    nd = wl.num_decode_tokens
    logits = _gpu_logits(wl)
    spans = ([(0, nd)] if nd else []) + ([(nd, wl.rows)] if nd < wl.rows else [])
    idx, cnt = [], []
    cpu = {n: getattr(wl, n).cpu() for n in ("visible", "positions", "seq_lens", "token_to_req",
                                              "block_table")}
    for lg, (a, b) in zip(logits, spans):
        i, c = oracle.topk_expand(lg, cpu["visible"][a:b], cpu["positions"][a:b],
                                  cpu["seq_lens"], cpu["token_to_req"][a:b],
                                  cpu["block_table"] if physical else None, s.width,
                                  s.compress_ratio, s.page_size, physical)
        idx.append(i)
        cnt.append(c)
    return torch.cat(idx), torch.cat(cnt)


@pytest.mark.gpu
@pytest.mark.parametrize("kv_layout,gate", [("token_major", False), ("head_major", True)])
def test_run_qsa_uniform_decode(kv_layout, gate):
    wl = make_workload("cpu_decode_4k", device=DEV, batch=6, kv_layout=kv_layout, gate=gate)
    print(f"[backend] uniform decode layout={kv_layout} gate={gate}", flush=True)
    layer, output = _run_layer(wl)
    want_idx, want_counts = _expected_selection(wl, physical=True)
    rows = wl.rows
    assert torch.equal(layer.topk_indices_buffer[:rows].cpu(), want_idx)
    assert torch.equal(layer.topk_counts_buffer[:rows].cpu(), want_counts)
    s = wl.shape
    kv = wl.kv_cache.cpu()
    if kv_layout == "token_major":
        k, v = kv[..., :s.head_dim], kv[..., s.head_dim:]
    else:
        k, v = kv.transpose(1, 2).split(s.head_dim, dim=-1)
    want = oracle.sparse_attention(wl.q.cpu(), k, v, want_idx, wl.block_table.cpu(),
                                   wl.token_to_req.cpu(), indices_are_physical=True,
                                   valid_counts=want_counts,
                                   output_gate=None if wl.gate is None else wl.gate.cpu())
    _check_attn(output[:rows], want, "uniform decode")
    assert (output[rows:].float() == 0).all(), "rows past num_actual_tokens are zeroed"


@pytest.mark.gpu
@pytest.mark.parametrize("decode_requests", [0, 3])
def test_run_qsa_prefill_and_mixed(decode_requests):
    """max_query_len > 1: logical ids for every row (decode rows included), no counts."""
    wl = make_workload("prefill_8k_on_16k", device=DEV, batch=5, chunk=40, prefix=0,
                       seq_len_min=700, seq_len_max=1500, seq_len_dist="uniform",
                       token_topk=256, decode_requests=decode_requests)
    print(f"[backend] prefill/mixed decode_requests={decode_requests} rows={wl.rows}", flush=True)
    layer, output = _run_layer(wl)
    want_idx, _ = _expected_selection(wl, physical=False)
    rows = wl.rows
    got_idx = layer.topk_indices_buffer[:rows].cpu()
    assert torch.equal(got_idx, want_idx)
    s = wl.shape
    kv = wl.kv_cache.cpu()
    want = oracle.sparse_attention(wl.q.cpu(), kv[..., :s.head_dim], kv[..., s.head_dim:],
                                   want_idx, wl.block_table.cpu(), wl.token_to_req.cpu())
    _check_attn(output[:rows], want, "prefill/mixed")
    assert (output[rows:].float() == 0).all()


@pytest.mark.gpu
@pytest.mark.parametrize("decode_requests", [0, 3])
def test_run_qsa_multi_token_decode(decode_requests):
    """decode_query_len = 2 (``attention.py:140``): request i owns decode rows
    2i and 2i + 1, scored by the decode scorer (``ops/indexer.py:241-279``);
    max_query_len = 2, so the plugin asks for logical ids and no counts
    (``attention.py:202-213``, ``backend.py:62-66``). ``decode_requests`` 0:
    a decode-only batch; 3: three decode requests, then ragged prefill chunks."""
    if decode_requests:
        wl = make_workload("prefill_8k_on_16k", device=DEV, batch=6, chunk=40, prefix=0,
                           seq_len_min=700, seq_len_max=1500, seq_len_dist="uniform",
                           token_topk=256, decode_requests=decode_requests, decode_query_len=2)
    else:
        wl = make_workload("cpu_decode_4k", device=DEV, batch=6, seq_len_min=3000,
                           seq_len_max=4096, seq_len_dist="uniform", decode_query_len=2)
    print(f"[backend] multi-token decode decode_requests={wl.num_decodes} rows={wl.rows} "
          f"decode rows={wl.num_decode_tokens}", flush=True)
    assert wl.max_query_len > 1 and wl.num_decode_tokens == 2 * wl.num_decodes
    layer, output = _run_layer(wl)
    want_idx, _ = _expected_selection(wl, physical=False)
    rows = wl.rows
    assert torch.equal(layer.topk_indices_buffer[:rows].cpu(), want_idx)
    s = wl.shape
    kv = wl.kv_cache.cpu()
    want = oracle.sparse_attention(wl.q.cpu(), kv[..., :s.head_dim], kv[..., s.head_dim:],
                                   want_idx, wl.block_table.cpu(), wl.token_to_req.cpu())
    _check_attn(output[:rows], want, "multi-token decode")
    assert (output[rows:].float() == 0).all()


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(12))
def test_select_random_batches(seed):
    """``select_paged_tokens`` on seeded random batches: decode-only (physical
    slots and counts) or decode requests of 1-3 rows followed by ragged prefill
    chunks (logical ids), top-k 256 or 512 tokens; bit-exact against the oracle
    on the kernels' own logits."""
    from qsa_vllm_amd.ops import select_paged_tokens
    g = torch.Generator().manual_seed(4000 + seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=g))]  # noqa: E731
    batch, dql, topk_tokens = pick([1, 2, 5, 8]), pick([1, 2, 3]), pick([256, 512])
    decode_requests = pick([0, batch // 2, batch])
    physical = decode_requests == batch
    if physical:
        wl = make_workload("cpu_decode_4k", device=DEV, batch=batch, seq_len_min=1500,
                           seq_len_max=6000, seq_len_dist="uniform", decode_query_len=dql,
                           token_topk=topk_tokens, seed=seed)
    else:
        wl = make_workload("prefill_8k_on_16k", device=DEV, batch=batch, chunk=pick([7, 33, 60]),
                           prefix=0, seq_len_min=600, seq_len_max=2500, seq_len_dist="uniform",
                           token_topk=topk_tokens, decode_requests=decode_requests,
                           decode_query_len=dql, seed=seed)
    s = wl.shape
    rows = wl.rows
    print(f"[backend] random select seed={seed} batch={batch} decodes={wl.num_decodes} dql={dql} "
          f"rows={rows} physical={physical}", flush=True)
    idx = torch.full((rows, s.width), -7, dtype=torch.int32, device=DEV)
    counts = torch.full((rows,), -7, dtype=torch.int32, device=DEV)
    select_paged_tokens(wl.q_index, wl.index_cache, wl.index_table, wl.token_to_req,
                        wl.positions, wl.seq_lens, s.token_topk, s.compress_ratio, idx,
                        query_start_loc=wl.query_start_loc, max_query_len=wl.max_query_len,
                        max_seq_len=wl.max_seq_len, num_decodes=wl.num_decodes,
                        num_decode_tokens=wl.num_decode_tokens, decode_query_len=dql,
                        main_block_table=wl.block_table if physical else None,
                        main_page_size=s.page_size,
                        valid_counts_out=counts if physical else None)
    want_idx, want_counts = _expected_selection(wl, physical=physical)
    assert torch.equal(idx.cpu(), want_idx)
    if physical:
        assert torch.equal(counts.cpu(), want_counts)


@pytest.mark.gpu
def test_select_multi_token_decode_physical():
    """``select_paged_tokens`` with decode_query_len = 2 and a main block table:
    physical slots and valid counts for both rows of every request, bit-exact
    against the oracle on the kernel's own logits; attention over them with the
    decode kernel."""
    from qsa_vllm_amd.ops import qsa_sparse_paged_attention, select_paged_tokens
    wl = make_workload("cpu_decode_4k", device=DEV, batch=5, seq_len_min=2000, seq_len_max=4096,
                       seq_len_dist="uniform", decode_query_len=2, seed=11)
    s = wl.shape
    rows = wl.rows
    print(f"[backend] multi-token decode physical rows={rows}", flush=True)
    idx = torch.full((rows, s.width), -7, dtype=torch.int32, device=DEV)
    counts = torch.full((rows,), -7, dtype=torch.int32, device=DEV)
    select_paged_tokens(wl.q_index, wl.index_cache, wl.index_table, wl.token_to_req,
                        wl.positions, wl.seq_lens, s.token_topk, s.compress_ratio, idx,
                        query_start_loc=wl.query_start_loc, max_query_len=2,
                        max_seq_len=wl.max_seq_len, num_decodes=wl.num_decodes,
                        num_decode_tokens=rows, decode_query_len=2,
                        main_block_table=wl.block_table, main_page_size=s.page_size,
                        valid_counts_out=counts)
    want_idx, want_counts = _expected_selection(wl, physical=True)
    assert torch.equal(idx.cpu(), want_idx)
    assert torch.equal(counts.cpu(), want_counts)
    out = qsa_sparse_paged_attention(wl.q, wl.k_cache, wl.v_cache, idx, wl.block_table,
                                     wl.token_to_req, use_decode_kernel=True,
                                     indices_are_physical=True, valid_counts=counts)
    torch.cuda.synchronize()
    want = oracle.sparse_attention(wl.q.cpu(), wl.k_cache.cpu(), wl.v_cache.cpu(), want_idx,
                                   wl.block_table.cpu(), wl.token_to_req.cpu(),
                                   indices_are_physical=True, valid_counts=want_counts)
    _check_attn(out, want, "multi-token decode, physical")


def _layer_step_case(prefix, chunk, seed):
    from qsa_vllm_amd.workloads import make_prepare_case
    return make_prepare_case(prefix, chunk, num_index_heads=8, index_head_dim=128,
                             compress_ratio=16, rotary_dim=64, main_kv_heads=2, main_head_dim=128,
                             main_page=16, device=DEV, seed=seed)


@pytest.mark.gpu
@pytest.mark.parametrize("prefix,chunk", [([300, 511, 700, 420], [1, 1, 1, 1]),
                                          ([40, 300], [48, 33])])
def test_layer_step_prepare_select_attend(prefix, chunk):
    """YuLanQSAIndexer.forward (prepare, then select) and YuLanQSAImpl.forward on one
    consistent state: the new tokens' keys and K/V written by prepare are what
    selection and attention read."""
    from types import SimpleNamespace
    from qsa_vllm_amd.graph_dispatch import decode_logits_columns, prefill_logits_width
    backend = _backend()
    case = _layer_step_case(prefix, chunk, seed=sum(chunk))
    topk, R, page, hq, d = 256, 16, 16, 16, 128
    width = topk + R - 1
    tokens = case.index_qk.shape[0]
    decode = max(chunk) == 1
    print(f"[backend] layer step prefix={prefix} chunk={chunk}", flush=True)
    # oracle first, on CPU copies of the untouched state
    cpu_args, kwargs = case.call_args()
    start = {k: v.cpu() for k, v in case.clone_outputs().items()}
    cpu_args = [a.cpu() if isinstance(a, torch.Tensor) else a for a in cpu_args]
    cpu_args[6] = SimpleNamespace(**{k: v.cpu() for k, v in vars(case.raw).items()})
    cpu_args[7] = SimpleNamespace(**{k: v.cpu() for k, v in vars(case.comp).items()})
    cpu_args[8], cpu_args[9] = start["state_cache"], start["compressed_cache"]
    cpu_args[12], cpu_args[13] = start["main_kv"][..., :d], start["main_kv"][..., d:]
    query_o = oracle.prepare(*cpu_args, **kwargs)

    indexer = backend.YuLanQSAIndexer(8, 128, R, topk, 64, 1.0e7, 1e-6, 8,
                                      case.state_cache, case.compressed_cache)
    indexer.q_layernorm.weight.data.copy_(case.q_norm_weight)
    indexer.k_layernorm.weight.data.copy_(case.k_norm_weight)
    indexer.cos_sin_cache = case.cos_sin
    layer = backend.QSALayerState(case.main_kv.permute(0, 2, 1, 3), d, tokens + 2, width)
    key_cache, value_cache = layer.main_kv_views()
    qsl = case.raw.query_start_loc
    comp_meta = backend.QSACompressedMetadata(
        block_table=case.comp_table, token_to_req=case.token_to_req,
        logical_positions=case.positions, seq_lens=case.seq_lens, query_start_loc=qsl,
        max_query_len=max(chunk), max_seq_len=int(case.seq_lens.max()),
        num_decodes=len(chunk) if decode else 0, num_decode_tokens=tokens if decode else 0,
        slot_mapping=case.comp.slot_mapping, k_work_metadata=case.comp.k_work_metadata)
    raw_meta = backend.QSARawMetadata(**vars(case.raw))
    indexer.forward(case.index_qk, case.positions, raw_meta, comp_meta,
                    layer.topk_indices_buffer[:tokens], case.main_key, case.main_value,
                    key_cache, value_cache, case.main_slots,
                    main_block_table=case.main_block_table if decode else None,
                    valid_counts_out=layer.topk_counts_buffer[:tokens] if decode else None)
    g = torch.Generator().manual_seed(5)
    q = (torch.randn(tokens, hq, d, generator=g)).to(torch.bfloat16).to(DEV)
    impl = backend.YuLanQSAImpl(hq, 2, d)
    main = backend.YuLanQSAMetadata(num_actual_tokens=tokens, max_query_len=max(chunk),
                                    block_table=case.main_block_table, slot_mapping=case.main_slots)
    output = torch.full((tokens + 2, hq, d), float("nan"), dtype=torch.bfloat16, device=DEV)
    impl.forward(layer, q, main, output, token_to_req=case.token_to_req)
    torch.cuda.synchronize()

    # caches written by prepare
    assert torch.equal(case.compressed_cache.cpu(), start["compressed_cache"])
    assert torch.equal(case.main_kv.cpu(), start["main_kv"])
    # selection: GPU scores of the oracle's prepared query, then the oracle's top-k
    visible = oracle.visible_blocks(case.positions.cpu(), case.seq_lens.cpu(),
                                    case.token_to_req.cpu(), R)
    cap = case.comp_table.shape[1] * case.compressed_cache.shape[1]
    if decode:
        cols = decode_logits_columns(int(case.seq_lens.max()), R, cap)
        lg = torch.full((tokens, cols), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_decode(query_o.to(DEV), case.compressed_cache,
                                                   case.comp_table, visible.to(DEV), lg, 1)
    else:
        cols = prefill_logits_width(int(case.seq_lens.max()), R, cap)
        lg = torch.full((tokens, cols), float("nan"), device=DEV)
        torch.ops.yulan_qsa_kernels.indexer_prefill(query_o.to(DEV), case.compressed_cache,
                                                    case.comp_table, qsl, visible.to(DEV), lg,
                                                    0, tokens, max(chunk))
    want_idx, want_cnt = oracle.topk_expand(lg.cpu(), visible, case.positions.cpu(),
                                            case.seq_lens.cpu(), case.token_to_req.cpu(),
                                            case.main_block_table.cpu() if decode else None,
                                            width, R, page, decode)
    assert torch.equal(layer.topk_indices_buffer[:tokens].cpu(), want_idx)
    if decode:
        assert torch.equal(layer.topk_counts_buffer[:tokens].cpu(), want_cnt)
    kv = start["main_kv"]
    want = oracle.sparse_attention(q.cpu(), kv[..., :d], kv[..., d:], want_idx,
                                   case.main_block_table.cpu(), case.token_to_req.cpu(),
                                   indices_are_physical=decode,
                                   valid_counts=want_cnt if decode else None)
    _check_attn(output[:tokens], want, "layer step")
    assert (output[tokens:].float() == 0).all()
