#!/usr/bin/env python
"""QSA decode benchmark on one MI355X.

Workload (the benchmark's headline shape, one GPU's TP2 share): decode batch 64,
context lengths uniform in [8192, 32768], 16 q / 2 kv heads x 128, bf16 paged KV
with 16-token pages, compress ratio 16, indexer 32 heads x 128, top-k 2048
tokens (128 pages) per query. A step is one QSA layer's decode path on that
batch: indexer scoring -> exact top-k + expansion to physical slots + counts ->
sparse paged attention (+ split merge). Inputs are resident in HBM.

Several query sets rotate across steps so successive steps select different
pages (the selected KV of all sets exceeds the 256 MB Infinity Cache). Steps
run from HIP graphs (one graph per block of steps) so host launch overhead is
not timed; K steps are timed with HIP events between two synchronisations.

The attention kernel's roofline figure comes from a separate timed loop of
attention-only graphs on the same stream: achieved = algorithmic bytes per
launch / mean launch time, against 8 TB/s. The CPU baseline times the eager
PyTorch oracle of the same path on this host on a bounded sample, for this
batch and for the small eager decode step (batch 4, 8 q / 1 kv heads, 4096
tokens).

The default line also carries compact figures of the plan's other workloads
(`workloads`: the same decode batch with page tables sized for a 524288-token
max-model-len, the long-context skewed decode batch, the chunked prefill) and
of the hybrid decoder step (`hybrid_step`); each has its own full line with
--workload NAME.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

METRIC = "QSA decode tokens/s + sparse-attn HBM GB/s (% of peak), 32k ctx, 1 MI355X"
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
WORKLOADS = ("decode_32k", "decode_32k_serving_width", "decode_long_skew", "prefill_8k_on_16k",
             "hybrid_decoder_step")


# CPU share of a one-GPU job on the benchmark hosts (worker pools are sized to it).
CPU_SHARE_PER_GPU = 16


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--workload", default="decode_32k", choices=WORKLOADS,
                   help="decode_32k is the headline; the others are secondary figures")
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--sets", type=int, default=4, help="query sets rotated across steps")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="CPU work budget for the oracle baseline (0 disables it)")
    p.add_argument("--cpu-threads", type=int, default=0,
                   help="0: the job's CPU share (16 per GPU on the benchmark hosts), at most the "
                        "CPUs this process may run on")
    p.add_argument("--no-extras", action="store_true",
                   help="headline workload only (no summaries of the other workloads)")
    p.add_argument("--no-hybrid", action="store_true",
                   help="decode_32k: skip the hybrid decoder step figures added to the line")
    p.add_argument("--traffic", default=os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                     "profiles", "select_attend_decode_32k_traffic.txt"),
                   help="committed rocprofv3 PMC summary giving HBM bytes per top-k + attention "
                        "launch")
    p.add_argument("--traffic-run", nargs="?", const="select_attend", default=None,
                   choices=("select_attend", "attention"),
                   help="no timing: eager launches of the workload's combined top-k + attention "
                        "op (or, with 'attention', of the sparse attention op alone over the "
                        "same selections) plus a calibration copy, for rocprofv3 --pmc "
                        "FETCH_SIZE / WRITE_SIZE passes")
    p.add_argument("--pmc-run", action="store_true",
                   help="no timing: three eager steps of the workload, for rocprofv3 --pmc runs")
    p.add_argument("--pmc-summary", metavar="DIR",
                   help="mean of every counter per QSA kernel over a rocprofv3 --pmc run")
    p.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                   help="summarise the counter CSVs of a FETCH_SIZE and a WRITE_SIZE pass of "
                        "--traffic-run and print the traffic summary")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def read_traffic(path):
    """HBM bytes per top-k + attention launch from the committed PMC summary, if present."""
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the QSA path is "
              "built and measured on a single MI355X.", file=sys.stderr)
        return 2
    if args.traffic_summary:
        print(traffic_summary(*args.traffic_summary))
        return 0
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary))
        return 0
    if args.steps <= 0:
        raise SystemExit("--steps must be positive")

    import torch

    from qsa_vllm_amd.workloads import make_workload

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "hybrid_decoder_step":
        return run_hybrid(args, dev)
    t0 = time.time()
    wl = make_workload(args.workload, device=dev)
    log(f"workload {args.workload} built in {time.time() - t0:.1f}s: rows={wl.rows} "
        f"kv_cache={wl.kv_cache.numel() * 2 / 1e9:.2f} GB")
    if not wl.is_decode:
        return run_prefill(args, wl)
    if args.traffic_run or args.pmc_run:
        return decode_counter_run(args, wl)
    m = measure_decode(wl, args.steps, args.warmup, args.sets, eager=True)
    s = wl.shape
    stream = torch.cuda.current_stream()
    # The committed counter summary covers the headline workload only.
    traffic = read_traffic(args.traffic) if args.workload == "decode_32k" else None
    result = {
        "metric": METRIC,
        "value": m["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["us_per_step"] * 1e-3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) activations and caches, permuted block tables",
        "config": {
            "workload": describe(s),
            "batch": s.batch,
            "query_sets": m["query_sets"],
            "kv_layout": s.kv_layout,
            "graph": "HIP graph per block of steps",
        },
        "roofline": dict(m["roofline"], traffic=traffic),
        "sparse_attention_roofline": m["sparse_attention_roofline"],
        "select_attend_fused": m["select_attend_fused"],
        "step_roofline": m["step_roofline"],
        "breakdown_us": m["breakdown_us"],
        "eager": m["eager"],
        "indexer_gbps": m["indexer_gbps"],
        "prepare": time_prepare(wl, stream),
        "layer_step": time_layer_step(wl, stream),
    }
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_baseline(wl, args)
        # The eager CPU decode step the benchmark plan names first (batch 4,
        # 8 q / 1 kv heads, 4096-token contexts), on the same cores.
        small = make_workload("cpu_decode_4k", device="cpu")
        result["cpu_baseline_cpu_decode_4k"] = cpu_baseline(small, args,
                                                            seconds=args.cpu_seconds / 2)
        del small
    if args.workload == "decode_32k" and not args.no_extras:
        # Every other workload of the plan beside the headline, compact (each
        # also has its own line: --workload NAME). A failure is recorded, not
        # raised, so it cannot take the headline figures with it.
        del wl
        result["workloads"] = {}
        for name in ("decode_32k_serving_width", "decode_long_skew", "prefill_8k_on_16k"):
            try:
                result["workloads"][name] = workload_summary(name, dev)
            except Exception as exc:  # noqa: BLE001
                result["workloads"][name] = {"error": f"{type(exc).__name__}: {exc}"}
            torch.cuda.empty_cache()
        if not args.no_hybrid:
            try:
                result["hybrid_step"] = hybrid_summary(dev)
            except Exception as exc:  # noqa: BLE001
                result["hybrid_step"] = {"error": f"{type(exc).__name__}: {exc}"}
    print(json.dumps(result), flush=True)
    return 0


def decode_queries(wl, n_sets):
    """The workload's (q, q_index) and n_sets - 1 fresh sets of the same shapes."""
    from qsa_vllm_amd.workloads import fresh_queries

    return [(wl.q, wl.q_index)] + [fresh_queries(wl, 100 + i) for i in range(n_sets - 1)]


def decode_counter_run(args, wl):
    """Eager decode steps for a rocprofv3 counter pass (no timing): scoring
    into logits, then the combined top-k + attention launch."""
    import torch

    from qsa_vllm_amd.graph_dispatch import decode_logits_columns
    from qsa_vllm_amd.ops import topk  # noqa: F401  (registers torch.ops.yulan_qsa_kernels)

    s, rows, dev = wl.shape, wl.rows, wl.device
    sets = decode_queries(wl, args.sets)
    idx = [torch.empty(rows, s.width, dtype=torch.int32, device=dev) for _ in sets]
    counts = [torch.empty(rows, dtype=torch.int32, device=dev) for _ in sets]
    out = torch.zeros_like(wl.q)
    cols = decode_logits_columns(wl.max_seq_len, s.compress_ratio,
                                 wl.index_table.shape[1] * wl.index_cache.shape[1])
    logits = [torch.empty(rows, cols, dtype=torch.float32, device=dev) for _ in sets]

    def score(i):
        torch.ops.yulan_qsa_kernels.indexer_decode(sets[i][1], wl.index_cache, wl.index_table,
                                                   wl.visible, logits[i], 1)

    def select_attend(i):
        torch.ops.yulan_qsa_kernels.decode_select_attend(
            logits[i], wl.visible, wl.positions, wl.seq_lens, wl.token_to_req, wl.block_table,
            idx[i], counts[i], s.compress_ratio, sets[i][0], wl.k_cache, wl.v_cache, out, None,
            0)

    def attend(i):
        torch.ops.yulan_qsa_kernels.sparse_attention(sets[i][0], wl.k_cache, wl.v_cache, idx[i],
                                                     wl.block_table, wl.token_to_req, out, None,
                                                     counts[i], True, 0)

    if args.traffic_run == "attention":
        # Selections by the top-k op (not in the summary's kernels), then the
        # attention alone.
        def select(i):
            score(i)
            torch.ops.yulan_qsa_kernels.topk_expand(logits[i], wl.visible, wl.positions,
                                                    wl.seq_lens, wl.token_to_req, wl.block_table,
                                                    idx[i], counts[i], s.compress_ratio,
                                                    s.page_size, True, True)

        return traffic_run(select, attend, len(sets))
    if args.traffic_run:
        return traffic_run(score, select_attend, len(sets))
    for _ in range(3):
        for i in range(len(sets)):
            score(i)
            select_attend(i)
    torch.cuda.synchronize()
    log(f"pmc run: {3 * len(sets)} eager decode steps")
    return 0


def measure_decode(wl, steps, warmup, n_sets, eager=False):
    """Decode steps of `wl` (indexer scoring -> top-k/expand + sparse attention,
    one op: decode_select_attend) from HIP graphs over n_sets rotating query
    sets, then each launch alone for the breakdown and the rooflines (the
    combined launch, and the standalone top-k and attention ops). Returns the
    figures as a dict (times in us)."""
    import torch

    from qsa_vllm_amd import _lib
    from qsa_vllm_amd.graph_dispatch import decode_logits_columns
    from qsa_vllm_amd.ops import decode_select_attend, qsa_sparse_paged_attention, topk_expand
    from qsa_vllm_amd.workloads import (attention_bytes, decode_step_bytes, indexer_bytes,
                                        topk_bytes)

    s = wl.shape
    rows = wl.rows
    dev = wl.device
    sets = decode_queries(wl, n_sets)
    n_sets = len(sets)
    idx = [torch.empty(rows, s.width, dtype=torch.int32, device=dev) for _ in sets]
    counts = [torch.empty(rows, dtype=torch.int32, device=dev) for _ in sets]
    outs = [torch.zeros_like(wl.q) for _ in sets]
    cols = decode_logits_columns(wl.max_seq_len, s.compress_ratio,
                                 wl.index_table.shape[1] * wl.index_cache.shape[1])
    logits = [torch.empty(rows, cols, dtype=torch.float32, device=dev) for _ in sets]
    fused = bool(_lib.load().qsa_decode_select_attention_fuses(
        rows, cols, s.width, s.compress_ratio, s.num_q_heads, s.num_kv_heads, s.head_dim)) and \
        s.kv_layout == "token_major"

    def step(i):
        decode_select_attend(sets[i][1], wl.index_cache, wl.index_table, wl.visible, sets[i][0],
                             wl.k_cache, wl.v_cache, wl.block_table, wl.token_to_req,
                             wl.positions, wl.seq_lens, s.token_topk, s.compress_ratio,
                             wl.max_seq_len, idx[i], counts[i], outs[i])

    def index_only(i):
        torch.ops.yulan_qsa_kernels.indexer_decode(sets[i][1], wl.index_cache, wl.index_table,
                                                   wl.visible, logits[i], 1)

    def select_attend_only(i):
        torch.ops.yulan_qsa_kernels.decode_select_attend(
            logits[i], wl.visible, wl.positions, wl.seq_lens, wl.token_to_req, wl.block_table,
            idx[i], counts[i], s.compress_ratio, sets[i][0], wl.k_cache, wl.v_cache, outs[i],
            None, 0)

    def topk_only(i):
        topk_expand(logits[i], wl.visible, wl.positions, wl.seq_lens, wl.token_to_req, idx[i],
                    s.compress_ratio, main_block_table=wl.block_table,
                    main_page_size=s.page_size, valid_counts_out=counts[i])

    def attend_only(i):
        qsa_sparse_paged_attention(sets[i][0], wl.k_cache, wl.v_cache, idx[i], wl.block_table,
                                   wl.token_to_req, outs[i], use_decode_kernel=True,
                                   indices_are_physical=True, valid_counts=counts[i])

    # Eager pass (also initialises allocator pools), then capture.
    for i in range(n_sets):
        index_only(i)
        topk_only(i)
        attend_only(i)
        select_attend_only(i)
        step(i)
    torch.cuda.synchronize()

    def capture(fn, indices):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in indices:
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in indices:
                fn(i)
        return g

    block_graph = capture(step, list(range(n_sets)))
    single = [capture(step, [i]) for i in range(n_sets)]
    reps = 8
    fused_graph = capture(select_attend_only, list(range(n_sets)) * reps)
    attn_graph = capture(attend_only, list(range(n_sets)) * reps)
    index_graph = capture(index_only, list(range(n_sets)) * reps)
    topk_graph = capture(topk_only, list(range(n_sets)) * reps)

    def run_steps(k):
        full, rest = divmod(k, n_sets)
        for _ in range(full):
            block_graph.replay()
        for i in range(rest):
            single[i].replay()

    stream = torch.cuda.current_stream()
    run_steps(warmup)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    run_steps(steps)
    stop.record(stream)
    torch.cuda.synchronize()
    us_step = start.elapsed_time(stop) * 1e3 / steps

    def time_graph(graph, launches, rounds):
        graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(rounds):
            graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / (launches * rounds)  # us per launch

    rounds = max(2, steps // (n_sets * reps))
    fused_us = time_graph(fused_graph, n_sets * reps, rounds)
    attn_us = time_graph(attn_graph, n_sets * reps, rounds)
    index_us = time_graph(index_graph, n_sets * reps, rounds)
    topk_us = time_graph(topk_graph, n_sets * reps, rounds)

    out = {}
    if eager:
        # The same steps launched eagerly (no graph): host launch overhead included.
        eager_steps = max(n_sets, (steps // n_sets) * n_sets)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for k in range(eager_steps):
            step(k % n_sets)
        b.record(stream)
        torch.cuda.synchronize()
        eager_us = a.elapsed_time(b) * 1e3 / eager_steps
        out["eager"] = {"us_per_step": round(eager_us, 3),
                        "tokens_per_s": round(rows / (eager_us * 1e-6), 1)}

    # Correctness gate on the timed data: counts follow the closed form.
    want_counts = s.token_topk + wl.seq_lens % s.compress_ratio
    for i in range(n_sets):
        if not torch.equal(counts[i], want_counts):
            raise SystemExit("valid counts differ from the closed form: results invalid")
        if not torch.isfinite(outs[i].float()).all():
            raise SystemExit("non-finite attention output: results invalid")

    attn_bytes = sum(attention_bytes(wl, counts[i]) for i in range(n_sets)) / n_sets
    attn_gbps = attn_bytes / (attn_us * 1e-6) / 1e9
    fused_bytes = attn_bytes + topk_bytes(wl)
    fused_gbps = fused_bytes / (fused_us * 1e-6) / 1e9
    step_bytes = sum(decode_step_bytes(wl, counts[i]) for i in range(n_sets)) / n_sets
    step_gbps = step_bytes / (us_step * 1e-6) / 1e9
    out.update({
        "query_sets": n_sets,
        "us_per_step": us_step,
        "tokens_per_s": round(rows / (us_step * 1e-6), 1),
        "select_attend_fused": fused,
        # The step's dominant launch: the row selection and the sparse
        # attention in one kernel (select_attend_kernel) plus the split merge,
        # or, for shapes the library does not fuse, the top-k and attention
        # launches it runs instead.
        "roofline": {
            "kernel": ("select_attend_kernel (top-k + sparse attention, + split merge)" if fused
                       else "topk + sparse_attn_kernel (+ split merge)"),
            "bound": "hbm",
            "achieved": round(fused_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(fused_gbps / HBM_PEAK_GBPS, 4),
            "algorithmic_bytes_per_launch": int(fused_bytes),
            "us_per_launch": round(fused_us, 3),
        },
        # The sparse attention op alone (qsa_sparse_paged_attention over the
        # same selections: the prefill rows' and unfused shapes' kernel).
        "sparse_attention_roofline": {
            "kernel": "sparse_attn_kernel (+ split merge)",
            "bound": "hbm",
            "achieved": round(attn_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(attn_gbps / HBM_PEAK_GBPS, 4),
            "algorithmic_bytes_per_launch": int(attn_bytes),
            "us_per_launch": round(attn_us, 3),
        },
        # The whole step (indexer + top-k + attention + merge, graph-replayed)
        # against the HBM time of its algorithmic bytes.
        "step_roofline": {
            "bound": "hbm",
            "achieved": round(step_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(step_gbps / HBM_PEAK_GBPS, 4),
            "algorithmic_bytes_per_step": int(step_bytes),
            "floor_us": round(step_bytes / (HBM_PEAK_GBPS * 1e3), 3),
            "us_per_step": round(us_step, 3),
        },
        "breakdown_us": {
            "indexer_decode": round(index_us, 3),
            "select_attend": round(fused_us, 3),
            "topk_expand_alone": round(topk_us, 3),
            "sparse_attention_alone": round(attn_us, 3),
            "step": round(us_step, 3),
        },
        "indexer_gbps": round(indexer_bytes(wl) / (index_us * 1e-6) / 1e9, 1),
        "logits_columns": cols,
    })
    return out


def workload_summary(name, dev, steps=40, warmup=8):
    """Compact figures of one more workload for the default benchmark line."""
    import torch

    from qsa_vllm_amd.workloads import make_workload

    wl = make_workload(name, device=dev)
    if wl.is_decode:
        m = measure_decode(wl, steps, warmup, 4)
        out = {"workload": describe(wl.shape), "rows": wl.rows,
               "tokens_per_s": m["tokens_per_s"], "us_per_step": round(m["us_per_step"], 3),
               "breakdown_us": m["breakdown_us"], "logits_columns": m["logits_columns"],
               "roofline": m["roofline"],
               "sparse_attention_roofline": m["sparse_attention_roofline"],
               "select_attend_fused": m["select_attend_fused"],
               "step_roofline": m["step_roofline"], "indexer_gbps": m["indexer_gbps"]}
    else:
        m = measure_prefill(wl, steps=5, warmup=2)
        out = {"workload": describe(wl.shape), "rows": wl.rows,
               "tokens_per_s": m["value"], "ms_per_step": m["ms_per_step"],
               "breakdown_ms": m["breakdown_ms"], "roofline": m["roofline"],
               "attention_gathered_gbps": m["attention_gathered_gbps"]}
    del wl
    torch.cuda.synchronize()
    return out


def time_prepare(wl, stream, rounds=20, reps=8):
    """qsa_prepare (index-q norm + RoPE, compression groups, ring commit, main
    K/V writes) for this step's tokens: decode rows append one token each,
    chunked prefill appends the chunk. Timed from a graph of `reps` launches."""
    import torch

    from qsa_vllm_amd.ops import qsa_prepare
    from qsa_vllm_amd.workloads import make_prepare_case

    s = wl.shape
    if wl.is_decode:
        prefix, chunk = (wl.seq_lens.cpu() - 1).tolist(), [1] * wl.rows
    else:
        prefix, chunk = [s.prefix] * s.batch, [s.chunk] * s.batch
    case = make_prepare_case(prefix, chunk, num_index_heads=s.index_heads,
                             index_head_dim=s.index_dim, compress_ratio=s.compress_ratio,
                             main_kv_heads=s.num_kv_heads, main_head_dim=s.head_dim,
                             main_page=s.page_size, history=False, device=wl.q.device,
                             seed=s.seed + 17)
    args, kwargs = case.call_args()
    qsa_prepare(*args, **kwargs)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        qsa_prepare(*args, **kwargs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            qsa_prepare(*args, **kwargs)
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(rounds):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / (rounds * reps)
    nbytes = case.prepare_bytes()
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"kernel": "prepare_kernel", "bound": "hbm", "tokens": case.index_qk.shape[0],
            "compression_groups": case.num_groups, "us_per_launch": round(us, 3),
            "algorithmic_bytes_per_launch": int(nbytes), "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4)}


def time_layer_step(wl, stream, reps=8, rounds=10):
    """The whole QSA decode layer step (prepare -> select -> attend) on the
    workload's caches and page tables, metadata from QSAMetadataBuilder, timed
    from a graph of `reps` back-to-back steps."""
    import torch

    from qsa_vllm_amd.backend import QSALayerState, YuLanQSAImpl, YuLanQSAIndexer
    from qsa_vllm_amd.graph_dispatch import SHORT_DECODE_COLUMNS, capture_column_scope
    from qsa_vllm_amd.layer_step import qsa_layer_step
    from qsa_vllm_amd.metadata import QSAMetadataBuilder

    s = wl.shape
    dev = wl.q.device
    rows = wl.rows
    ring = torch.zeros(rows + 2, s.compress_ratio, s.index_dim, dtype=torch.bfloat16, device=dev)
    indexer = YuLanQSAIndexer(s.index_heads, s.index_dim, s.compress_ratio, s.token_topk, 64,
                              1.0e7, 1e-6, int(wl.seq_lens.max()) + 1, ring, wl.index_cache)
    kv_view = wl.kv_cache.permute(0, 2, 1, 3) if s.kv_layout == "token_major" else wl.kv_cache
    layer = QSALayerState(kv_view, s.head_dim, rows, s.width)
    impl = YuLanQSAImpl(s.num_q_heads, s.num_kv_heads, s.head_dim)
    builder = QSAMetadataBuilder(
        compress_ratio=s.compress_ratio, main_page_size=s.page_size,
        comp_page_size=wl.index_cache.shape[1], ring_size=s.compress_ratio,
        max_num_requests=rows, max_num_tokens=rows, main_table_width=wl.block_table.shape[1],
        comp_table_width=wl.index_table.shape[1], device=dev)
    batch = builder.build((wl.seq_lens.cpu() - 1).tolist(), [1] * rows, wl.block_table,
                          wl.index_table, torch.arange(rows, dtype=torch.int32))
    idx_cols, kv_cols = (s.index_heads + 1) * s.index_dim, s.num_kv_heads * s.head_dim
    gen = torch.Generator(device=dev).manual_seed(s.seed + 23)
    projected = (torch.randn(rows, idx_cols + 2 * kv_cols, generator=gen, device=dev)
                 * 0.5).to(torch.bfloat16)
    index_qk = projected[:, :idx_cols]
    main_key = projected[:, idx_cols:idx_cols + kv_cols].view(rows, s.num_kv_heads, s.head_dim)
    main_value = projected[:, idx_cols + kv_cols:].view(rows, s.num_kv_heads, s.head_dim)
    output = torch.empty_like(wl.q)

    def step():
        qsa_layer_step(indexer, impl, layer, batch, index_qk, main_key, main_value, wl.q, output)

    with capture_column_scope(SHORT_DECODE_COLUMNS):
        step()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                step()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(rounds):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    if not torch.isfinite(output.float()).all():
        raise SystemExit("non-finite layer step output: results invalid")
    us = a.elapsed_time(b) * 1e3 / (rounds * reps)
    return {"ops": "qsa_prepare -> select_paged_tokens -> qsa_sparse_paged_attention",
            "us_per_step": round(us, 3), "tokens_per_s": round(rows / (us * 1e-6), 1)}


def describe(s):
    if s.seq_len_dist == "uniform":
        ctx = f"context U[{s.seq_len_min},{s.seq_len_max}]"
    elif s.seq_len_dist == "lognormal":
        ctx = (f"context lognormal(median {s.lognormal_median:.0f}, sigma {s.lognormal_sigma}) "
               f"clipped to [{s.seq_len_min},{s.seq_len_max}]")
    else:
        ctx = f"context {s.seq_len_min}"
    kind = (f"chunked prefill {s.batch} x {s.chunk} new tokens on a {s.prefix}-token prefix"
            if s.chunk else f"decode batch {s.batch}")
    return (f"{s.name}: {kind}, {ctx}, {s.num_q_heads}q/{s.num_kv_heads}kv x {s.head_dim}, "
            f"page {s.page_size}, compress ratio {s.compress_ratio}, top-k {s.token_topk} "
            f"tokens, indexer {s.index_heads}x{s.index_dim}")


def run_prefill(args, wl):
    """Chunked prefill step: prefill scoring (MFMA) -> logical top-k/expand ->
    sparse attention over logical ids. The step's rows are the new tokens."""
    if args.pmc_run:
        measure_prefill(wl, 3, 0, pmc_run=True)
        return 0
    result = measure_prefill(wl, max(1, min(args.steps, 20)), min(args.warmup, 3))
    print(json.dumps(result), flush=True)
    return 0


def measure_prefill(wl, steps, warmup, pmc_run=False):
    """The chunked-prefill step's figures (see run_prefill) as a dict."""
    import torch

    from qsa_vllm_amd.graph_dispatch import prefill_logits_width
    from qsa_vllm_amd.ops import qsa_sparse_paged_attention, select_paged_tokens, topk_expand
    from qsa_vllm_amd.workloads import indexer_flops

    s = wl.shape
    rows = wl.rows
    dev = wl.device
    idx = torch.empty(rows, s.width, dtype=torch.int32, device=dev)
    out = torch.zeros_like(wl.q)
    width = prefill_logits_width(wl.max_seq_len, s.compress_ratio,
                                 wl.index_table.shape[1] * wl.index_cache.shape[1])
    # The indexer and top-k figures cover the same logits spans as the step
    # (select_paged_tokens caps the logits buffer and the library sizes spans).
    from qsa_vllm_amd import _lib
    from qsa_vllm_amd.ops.indexer import _LOGITS_CAP_BYTES
    span = max(1, int(_lib.load().qsa_indexer_prefill_span_rows(width, _LOGITS_CAP_BYTES)))
    spans = [(a, min(rows, a + span)) for a in range(0, rows, span)]
    logits = torch.empty(min(rows, span), width, dtype=torch.float32, device=dev)

    def select():
        select_paged_tokens(wl.q_index, wl.index_cache, wl.index_table, wl.token_to_req,
                            wl.positions, wl.seq_lens, s.token_topk, s.compress_ratio, idx,
                            query_start_loc=wl.query_start_loc, max_query_len=wl.max_query_len,
                            max_seq_len=wl.max_seq_len, visible_blocks=wl.visible)

    def attend():
        qsa_sparse_paged_attention(wl.q, wl.k_cache, wl.v_cache, idx, wl.block_table,
                                   wl.token_to_req, out)

    def index_only():
        for a, b in spans:
            torch.ops.yulan_qsa_kernels.indexer_prefill(wl.q_index, wl.index_cache,
                                                        wl.index_table, wl.query_start_loc,
                                                        wl.visible, logits[:b - a], a, b - a,
                                                        wl.max_query_len)

    def topk_only():
        for a, b in spans:
            topk_expand(logits[:b - a], wl.visible[a:b], wl.positions[a:b], wl.seq_lens,
                        wl.token_to_req[a:b], idx[a:b], s.compress_ratio)

    def step():
        select()
        attend()

    if pmc_run:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        log(f"pmc run: {steps} eager prefill steps")
        return None

    stream = torch.cuda.current_stream()

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps  # ms

    for _ in range(warmup):
        step()
    ms_step = timed(step, steps)
    idx_ms = timed(index_only, steps)
    topk_ms = timed(topk_only, steps)
    attn_ms = timed(attend, steps)
    if not torch.isfinite(out.float()).all():
        raise SystemExit("non-finite attention output: results invalid")
    flops = indexer_flops(wl)
    valid = int((idx >= 0).sum())
    gathered = valid * s.num_kv_heads * 2 * s.head_dim * 2
    tflops = flops / (idx_ms * 1e-3) / 1e12
    result = {
        "metric": f"QSA chunked-prefill new tokens/s + prefill indexer bf16 TFLOP/s, 1 MI355X",
        "value": round(rows / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) activations and caches, permuted block tables",
        "config": {"workload": describe(s), "rows": rows},
        "roofline": {
            "kernel": "indexer_prefill_kernel",
            "bound": "mfma",
            "achieved": round(tflops, 1),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
            "traffic": None,
            "algorithmic_flops_per_step": flops,
            "launches_per_step": len(spans),
            "ms_per_step": round(idx_ms, 4),
        },
        "breakdown_ms": {
            "indexer_prefill": round(idx_ms, 4),
            "topk_expand": round(topk_ms, 4),
            "sparse_attention": round(attn_ms, 4),
            "step": round(ms_step, 4),
        },
        "attention_gathered_gbps": round(gathered / (attn_ms * 1e-3) / 1e9, 1),
        "attention_gathered_bytes": gathered,
        "prepare": time_prepare(wl, stream, rounds=5, reps=4),
    }
    return result




def hybrid_workload(dev, seed=11):
    """The hybrid decoder's mixed continuous batch (112 decode requests at
    contexts U[4096, 32768], 16 prefill chunks of 512 tokens)."""
    from qsa_vllm_amd.hybrid import make_serving_hybrid_workload

    return make_serving_hybrid_workload(dev, seed=seed)


def hybrid_flops(wl):
    """Projection/MLP GEMM FLOPs of one step (2 per weight per token) plus the
    LM head rows."""
    cfg, m = wl.cfg, wl.model
    tokens = wl.num_tokens
    per_token = 0
    for layer in m.layers:
        mx = layer.mixer
        mats = [layer.mlp.gate_up_proj, layer.mlp.down_proj]
        for norm in (layer.input_layernorm, layer.post_attention_layernorm):
            mats += [norm.gate_down, norm.gate_up]
        if layer.kind == "full_attention":
            mats += [mx.qkv_weight, mx.o_proj]
        else:
            mats += [mx.in_proj_qkvz, mx.in_proj_ba, mx.out_proj]
        per_token += sum(w.numel() for w in mats)
    per_token += m.norm.gate_down.numel() + m.norm.gate_up.numel()
    return 2 * per_token * tokens + 2 * m.lm_head.numel() * len(wl.scheduled)


def measure_hybrid(dev, steps, warmup, breakdown=True):
    """Times whole hybrid decoder steps (metadata build, embedding, 32 layers,
    final norm, LM-head rows) on the mixed batch; eager launches (a mixed batch
    is not captured). Returns the figures as a dict."""
    import torch

    from qsa_vllm_amd.gemm_tuning import disable_tuned_gemms, enable_tuned_gemms

    tuned = enable_tuned_gemms()
    log(f"library GEMM choices from the recorded tuning file: {tuned}")
    t0 = time.time()
    wl = hybrid_workload(dev)
    model = wl.model
    torch.cuda.synchronize()
    log(f"hybrid workload built in {time.time() - t0:.1f}s: tokens={wl.num_tokens} "
        f"requests={len(wl.scheduled)} memory={torch.cuda.memory_allocated() / 2**30:.1f} GiB")

    def step():
        return model.forward(wl.build())

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall = time.time()
    a.record(stream)
    for _ in range(steps):
        logits = step()
    b.record(stream)
    torch.cuda.synchronize()
    wall = (time.time() - wall) / steps * 1e3
    ms_step = a.elapsed_time(b) / steps
    if not torch.isfinite(logits).all():
        raise SystemExit("non-finite logits: results invalid")
    parts = {}
    if breakdown:
        # Per-part times from one more step with events between the parts.
        batch = wl.build()
        marks = []

        def mark(name):
            e = torch.cuda.Event(enable_timing=True)
            e.record(stream)
            marks.append((name, e))

        mark("start")
        hidden, residual = model.embed(batch.token_ids), None
        for layer in model.layers:
            if residual is None:
                residual = hidden
                normalized = layer.input_layernorm(hidden)
            else:
                normalized, residual = layer.input_layernorm(hidden, residual)
            mark("norms")
            hidden = layer.mixer(normalized, batch)
            mark("qsa_mixer" if layer.kind == "full_attention" else "gdn_mixer")
            normalized, residual = layer.post_attention_layernorm(hidden, residual)
            mark("norms")
            hidden = layer.mlp(normalized)
            mark("mlp")
        model.logits(hidden, residual, batch)
        mark("head")
        torch.cuda.synchronize()
        for (_, e0), (name, e1) in zip(marks, marks[1:]):
            parts[name] = parts.get(name, 0.0) + e0.elapsed_time(e1)
    flops = hybrid_flops(wl)
    out = {"wl": wl, "ms_per_step": ms_step, "wall_ms_per_step": wall, "flops": flops,
           "breakdown_ms": {k: round(v, 3) for k, v in parts.items()},
           "decode_graph": measure_hybrid_decode_graph(wl, steps=max(steps, 5)),
           "tuned_gemms": tuned}
    disable_tuned_gemms()
    return out


def measure_hybrid_decode_graph(wl, steps):
    """The model's uniform decode step over the workload's decode requests
    (one token each), replayed from a HIP graph: per step, a metadata build
    (host inputs to the persistent buffers) and one replay."""
    import torch

    from qsa_vllm_amd.hybrid import HybridDecodeGraph

    graph = HybridDecodeGraph(wl.model, wl.build_decode())
    for _ in range(2):
        graph.replay(wl.build_decode())
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        graph.replay(wl.build_decode())
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    a.record(stream)
    for _ in range(steps):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    replay_ms = a.elapsed_time(b) / steps
    n = graph.num_tokens
    del graph
    return {"requests": n, "ms_per_step": round(ms, 3), "replay_only_ms": round(replay_ms, 3),
            "tokens_per_s": round(n / (ms * 1e-3), 1)}


def hybrid_description(wl):
    from qsa_vllm_amd.hybrid import SERVING_CHUNK, SERVING_CHUNKS, SERVING_DECODES

    cfg = wl.cfg
    kinds = [layer.kind for layer in wl.model.layers]
    return (f"hybrid decoder step: {cfg.num_layers} layers ({kinds.count('linear_attention')} GDN, "
            f"{kinds.count('full_attention')} QSA), hidden {cfg.hidden_size}, TP{cfg.tp_size} share: "
            f"QSA {cfg.heads}q/{cfg.kv_heads}kv x {cfg.head_dim}, GDN {cfg.key_heads}k/"
            f"{cfg.value_heads}v heads x {cfg.linear_key_head_dim}, MLP {cfg.intermediate}, vocab "
            f"shard {cfg.vocab_shard}; batch {SERVING_DECODES} decode (context U[4096,32768]) + "
            f"{SERVING_CHUNKS} prefill chunks of {SERVING_CHUNK}")


def hybrid_summary(dev):
    """Compact hybrid-step figures for the default benchmark line."""
    m = measure_hybrid(dev, steps=3, warmup=2)
    wl = m.pop("wl")
    out = {"workload": hybrid_description(wl), "tokens": wl.num_tokens,
           "ms_per_step": round(m["ms_per_step"], 3),
           "tokens_per_s": round(wl.num_tokens / (m["ms_per_step"] * 1e-3), 1),
           "gemm_tflops": round(m["flops"] / (m["ms_per_step"] * 1e-3) / 1e12, 1),
           "breakdown_ms": m["breakdown_ms"], "decode_graph": m["decode_graph"],
           "library_gemm_choices": "recorded tuning file" if m["tuned_gemms"] else "library default"}
    del wl
    return out


def run_hybrid(args, dev):
    """The hybrid decoder step as the benchmark's own line."""
    import torch

    if args.pmc_run:
        wl = hybrid_workload(dev)
        for _ in range(2):
            wl.model.forward(wl.build())
        torch.cuda.synchronize()
        log("pmc run: 2 eager hybrid steps")
        return 0
    warmup = max(1, min(args.warmup, 3))
    steps = max(1, min(args.steps, 10))
    m = measure_hybrid(dev, steps, warmup)
    wl = m["wl"]
    ms_step = m["ms_per_step"]
    tflops = m["flops"] / (ms_step * 1e-3) / 1e12
    result = {
        "metric": "hybrid decoder step tokens/s (32 layers, 3 GDN : 1 QSA, 112 decode + 16 x 512 "
                  "prefill), 1 MI355X",
        "value": round(wl.num_tokens / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 3),
        "wall_ms_per_step": round(m["wall_ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init bf16 weights N(0, 0.02), seeded token ids, random "
                "cache and GDN-state history",
        "config": {"workload": hybrid_description(wl), "tokens": wl.num_tokens,
                   "requests": len(wl.scheduled), "graph": "eager",
                   "library_gemm_choices": ("recorded tuning file" if m["tuned_gemms"]
                                            else "library default")},
        "roofline": {
            "kernel": "whole step (projection, MLP and LM head GEMMs)",
            "bound": "mfma",
            "achieved": round(tflops, 1),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
            "traffic": None,
            "algorithmic_flops_per_step": m["flops"],
        },
        "breakdown_ms": m["breakdown_ms"],
        "decode_graph": m["decode_graph"],
    }
    print(json.dumps(result), flush=True)
    return 0


# Calibration copy for the counter passes: an fp32 negation (reads and writes
# CAL_BYTES once each), recognised in the counter CSV by its kernel name.
CAL_BYTES = 256 << 20
CAL_KERNEL = "neg_kernel"
# The decode step's dominant launch (the combined top-k + attention kernel) or
# the sparse attention kernel alone, and the split merge.
ATTN_KERNELS = ("select_attend_kernel", "sparse_attn_kernel", "merge_kernel")


def traffic_run(prepare, launch, n_sets, rounds=3):
    """prepare(i) for every set, then `rounds` passes of launch(i), whose
    kernels the counter summary reads."""
    import torch

    for i in range(n_sets):
        prepare(i)
    torch.cuda.synchronize()
    for _ in range(rounds):
        for i in range(n_sets):
            launch(i)
    src = torch.ones(CAL_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(rounds):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    log(f"traffic run: {rounds * n_sets} top-k + attention launches, {rounds} calibration copies "
        f"of {CAL_BYTES} B")
    return 0


def _counter_means(root, counter):
    """Mean counter value per dispatch, by kernel group, over a rocprofv3 --pmc run."""
    import csv
    import glob

    files = glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {root}")
    per_dispatch = {}
    for path in files:
        with open(path) as fh:
            for rec in csv.DictReader(fh):
                if rec.get("Counter_Name") != counter:
                    continue
                name = rec["Kernel_Name"]
                group = next((k for k in ATTN_KERNELS + (CAL_KERNEL,) if k in name), None)
                if group is None:
                    continue
                key = (path, rec["Dispatch_Id"])
                grp, val = per_dispatch.get(key, (group, 0.0))
                per_dispatch[key] = (grp, val + float(rec["Counter_Value"]))
    sums, counts = {}, {}
    for grp, val in per_dispatch.values():
        sums[grp] = sums.get(grp, 0.0) + val
        counts[grp] = counts.get(grp, 0) + 1
    return {g: (sums[g] / counts[g], counts[g]) for g in sums}


QSA_KERNELS = ("select_attend_kernel", "sparse_attn_kernel", "merge_kernel", "topk_direct_kernel",
               "topk_adaptive_kernel", "topk_partition_kernel", "topk_merge_kernel",
               "indexer_decode_kernel", "indexer_prefill_kernel")


def pmc_summary(root):
    """Mean value per dispatch of every collected counter, per QSA kernel."""
    import csv
    import glob

    files = glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {root}")
    per = {}  # (kernel, counter) -> {dispatch: value}
    for path in files:
        with open(path) as fh:
            for rec in csv.DictReader(fh):
                name = next((k for k in QSA_KERNELS if k in rec["Kernel_Name"]), None)
                if name is None:
                    continue
                d = per.setdefault((name, rec["Counter_Name"]), {})
                key = (path, rec["Dispatch_Id"])
                d[key] = d.get(key, 0.0) + float(rec["Counter_Value"])
    lines = []
    for (name, counter), d in sorted(per.items()):
        vals = list(d.values())
        lines.append(f"{name} {counter}: mean {sum(vals) / len(vals):.6g} over {len(vals)} dispatches")
    return "\n".join(lines)


def traffic_summary(fetch_dir, write_dir):
    """HBM bytes per combined launch (top-k + attention kernel + split merge), each
    counter scaled by what it reads for the calibration copy of CAL_BYTES."""
    fetch = _counter_means(fetch_dir, "FETCH_SIZE")
    write = _counter_means(write_dir, "WRITE_SIZE")
    for table, name in ((fetch, "FETCH_SIZE"), (write, "WRITE_SIZE")):
        missing = [k for k in (CAL_KERNEL,) if k not in table]
        if not any(k in table for k in ATTN_KERNELS[:2]):
            missing.append(" or ".join(ATTN_KERNELS[:2]))
        if missing:
            raise SystemExit(f"{name} pass lacks dispatches of {missing}")
    f_scale = CAL_BYTES / (fetch[CAL_KERNEL][0] * 1024.0)
    w_scale = CAL_BYTES / (write[CAL_KERNEL][0] * 1024.0)
    lines = [f"calibration: fp32 negation of {CAL_BYTES} B reads FETCH_SIZE "
             f"{fetch[CAL_KERNEL][0]:.1f} KiB, WRITE_SIZE {write[CAL_KERNEL][0]:.1f} KiB "
             f"-> scale fetch x{f_scale:.4f}, write x{w_scale:.4f}"]
    total = 0.0
    for k in ATTN_KERNELS:
        if k not in fetch:
            continue
        fb = fetch[k][0] * 1024.0 * f_scale
        wb = write.get(k, (0.0, 0))[0] * 1024.0 * w_scale
        total += fb + wb
        lines.append(f"{k}: {fetch[k][1]} dispatches, fetch {fb / 1e6:.2f} MB, "
                     f"write {wb / 1e6:.2f} MB per dispatch (scaled)")
    lines.append(f"traffic_bytes_per_launch: {total:.0f}")
    return "\n".join(lines)


def cpu_baseline(wl, args, seconds=None):
    """Eager-PyTorch oracle of the same decode step on this host's cores."""
    import torch

    import oracle

    seconds = args.cpu_seconds if seconds is None else seconds
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = args.cpu_threads or min(CPU_SHARE_PER_GPU, usable or 1)
    torch.set_num_threads(threads)
    cpu = {n: getattr(wl, n).cpu() for n in ("q", "q_index", "index_cache", "index_table",
                                             "block_table", "positions", "seq_lens")}
    kv = wl.kv_cache.cpu()
    d = wl.shape.head_dim
    k_cache, v_cache = kv[..., :d], kv[..., d:]
    steps = 0
    t0 = time.perf_counter()
    while True:
        oracle.decode_step(cpu["q_index"], cpu["index_cache"], cpu["index_table"], cpu["q"],
                           k_cache, v_cache, cpu["block_table"], cpu["positions"],
                           cpu["seq_lens"], wl.shape.token_topk, wl.shape.compress_ratio)
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return {
        "value": round(steps * wl.rows / elapsed, 2),
        "unit": "tokens/s",
        "cores": threads,
        "host_cpus": os.cpu_count(),
        "threads_note": _threads_note(threads, usable, args.cpu_threads),
        "kind": "port",
        "sample": f"{steps} full decode step(s) of the {wl.shape.name} batch ({wl.rows} rows) in "
                  f"{elapsed:.1f}s: oracle indexer -> top-k/expand -> fp32 sparse attention",
        "cpu": _cpu_model(),
        "torch": torch.__version__,
    }


def _threads_note(threads, usable, requested):
    if requested:
        return f"{threads} threads set by --cpu-threads"
    if usable and usable > CPU_SHARE_PER_GPU:
        return (f"{threads} of the {usable} CPUs this process may run on: the CPU share of a "
                f"one-GPU job on the benchmark hosts")
    return f"every CPU this process may run on ({threads})"


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
