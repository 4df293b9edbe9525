"""Decode throughput of the sparse-attention hot path on one MI355X.

Workload: one CSA2 attention layer decoding one token per row for
B=32 rows at context 32768: bf16 queries, 128 heads over the shared 512+64 latent stored
as FP8-b128 (656 B/entry), FP8 lightning indexer 64x128 over the 8192 compressed entries
(ratio 4), top-2048, sliding window 128, per-head sink.  A "step" is one replay of a HIP
graph holding ``SparseDecodeLayer.step`` of --layers (default 8) consecutive layers, each
with its own caches and inputs, as a model's decode graph holds its layers: per layer the
window append, indexer-query quantization, indexer scores, top-k, sparse MQA (split-KV) and
the split merge.  Distinct layers keep one layer's working set (about 90 MB) from being
served out of the last-level cache on the next step.  value = B x layers / replay time
(token-rows through one attention layer per second); ms_per_step is per layer.  Inputs are
synthetic (seeds 1..layers) and resident in HBM before timing starts.

Prints one JSON line (metric, value = decode tokens/s on this GPU, roofline of the
dominant kernel measured with HIP events on its stream, cpu_baseline = the CPU oracle's
decode step on this host's cores over the same workload).
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import re
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0

# Algorithmic work per decoded row
ENTRY_BYTES = 656                 # FP8-b128 latent entry
QO_BYTES = 2 * 128 * 576 * 2      # q read + out written, bf16
IDX_KEY_BYTES = 132               # FP8 indexer key (128 codes + fp32 scale)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--nsplit", type=int, default=4)
    ap.add_argument("--layers", type=int, default=8, help="distinct attention layers in the replayed graph")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline time budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--stage-iters", type=int, default=0, help="launches per stage timing (0: max(steps, 50))")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (3 launches): the reference kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    return ap.parse_args()


def build_layer(torch, dev, nsplit, seed=1):
    from mzoo_amd.decode import DecodeConfig, SparseDecodeLayer
    cfg = DecodeConfig(batch=32, heads=128, nope=512, rope=64, index_heads=64, index_dim=128, ratio=4, window=128,
                       topk=2048, max_groups=8192, index_format="fp8", nsplit=nsplit)
    ctx = 32768
    gen = torch.Generator(device=dev).manual_seed(seed)
    sinks = torch.randn(cfg.heads, generator=gen, device=dev)
    layer = SparseDecodeLayer(cfg, dev, sinks=sinks)
    b, d = cfg.batch, cfg.dim
    layer.fill_window(torch.randn(b, cfg.window, d, generator=gen, device=dev).bfloat16(), ctx - 2)
    layer.append_groups(0, torch.randn(b, cfg.max_groups, d, generator=gen, device=dev).bfloat16(),
                        torch.randn(b, cfg.max_groups, cfg.index_dim, generator=gen, device=dev).bfloat16())
    layer.set_positions(ctx - 1)
    q = torch.randn(b, cfg.heads, d, generator=gen, device=dev).bfloat16()
    kv = torch.randn(b, d, generator=gen, device=dev).bfloat16()
    q_idx = torch.randn(b, cfg.index_heads, cfg.index_dim, generator=gen, device=dev).bfloat16()
    w = torch.randn(b, cfg.index_heads, generator=gen, device=dev) * cfg.index_heads ** -0.5
    return layer, (q, kv, q_idx, w), sinks


def time_launches(torch, fn, iters):
    """Average duration of `fn` (its kernels on the current stream), HIP events."""
    st = torch.cuda.current_stream()
    fn()
    st.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(iters):
        fn()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters * 1e3  # microseconds


def capture_layers(torch, layers, inputs):
    """One HIP graph over the decode steps of several layers (static copies of the inputs);
    warm-up on a side stream first, as ``SparseDecodeLayer.capture`` does for one layer."""
    statics = [tuple(t.clone() for t in inp) for inp in inputs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for layer, st in zip(layers, statics):
                layer.step(*st)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for layer, st in zip(layers, statics):
            layer.step(*st)
    return g, statics


def stage_times(torch, layers, inputs, iters):
    """Average duration of each kernel of the step alone: a HIP graph of back-to-back
    launches of that kernel cycling through the layers (consecutive launches read different
    caches, as in the decode graph), replayed and timed with HIP events on the stream the
    kernels run on.  Inside a graph the launches follow each other with no host gap, so the
    figure is the kernel's own duration."""
    per_layer = [stage_fns(torch, layer, inp) for layer, inp in zip(layers, inputs)]
    nl = len(per_layer)
    reps = max(1, (32 + nl - 1) // nl)  # at least 32 launches per replay (amortizes the replay launch)
    replays = max(1, iters // (reps * nl))
    out = {}
    for name in per_layer[0]:
        fns = [d[name] for d in per_layer]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for f in fns:
                f()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                for f in fns:
                    f()
        out[name] = time_launches(torch, g.replay, replays) / (reps * nl)
    return out


def stage_fns(torch, layer, inputs):
    """The step's launches for one layer, each callable alone."""
    from mzoo_amd import _lib, indexer
    cfg = layer.cfg
    b = cfg.batch
    q, kv, q_idx, w = inputs
    ws = layer.workspace
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def indexer_decode():
        # window append + indexer-query quantization + FP8 scores: the step's first launch
        _lib.call("mzk_indexer_decode_fp8", q_idx.data_ptr(), w.data_ptr(), layer.k_codes.data_ptr(),
                  layer.k_scales.data_ptr(), b, cfg.index_heads, cfg.index_dim, cfg.max_groups, cfg.max_groups,
                  layer.positions.data_ptr(), cfg.ratio, layer.scores.data_ptr(), cfg.max_groups, None, None,
                  kv.data_ptr(), cfg.nope, cfg.rope, layer.win.data_ptr(), cfg.window, cfg.window, st())

    def attn():
        # the split-KV attention kernel alone: with no `out` the entry point writes the
        # split partials into the workspace and launches nothing else
        _lib.call("mzk_sparse_mqa", q.data_ptr(), b, 1, cfg.heads, cfg.dim, 1, cfg.nope, layer.positions.data_ptr(),
                  layer.win.data_ptr(), cfg.window, cfg.window, cfg.window, None, 0, 0, 1, layer.main.data_ptr(),
                  cfg.max_groups, cfg.max_groups, layer.idx.data_ptr(), cfg.topk, cfg.topk,
                  layer.sinks.data_ptr(), cfg.nsplit, ws.data_ptr(), ws.numel() * ws.element_size(), None, None, st())

    def combine():
        _lib.call("mzk_sparse_mqa_combine", ws.data_ptr(), b, 1, cfg.heads, cfg.dim, cfg.nsplit,
                  layer.sinks.data_ptr(), layer.out.data_ptr(), layer.lse.data_ptr(), st())

    return {
        "indexer_decode_fp8": indexer_decode,
        "topk": lambda: indexer.topk(layer.scores.view(b, cfg.max_groups), cfg.topk, out=layer.idx),
        "sparse_mqa": attn,
        "sparse_mqa_combine": combine,
    }


def cpu_baseline(torch, layer, inputs, budget_s):
    """The CPU oracle's decode step (indexer scores -> top-k -> attention) in fp32 on the
    dequantized caches, all 32 rows, on this host's cores; median of repeated steps."""
    from mzoo_amd import quant
    from oracle import attention as OA
    from oracle import quant as OQ
    cfg = layer.cfg
    q, kv, q_idx, w = (t.float().cpu() for t in inputs)
    win = quant.unpack_latent_fp8_b128(layer.win, dtype=torch.float32).cpu()
    main = quant.unpack_latent_fp8_b128(layer.main, dtype=torch.float32).cpu()
    kd = (layer.k_codes.cpu().view(torch.float8_e4m3fn).float() * layer.k_scales.cpu().unsqueeze(-1))
    sinks = layer.sinks.cpu()
    pos = int(layer.positions[0])
    positions = torch.full((cfg.batch, 1), pos, dtype=torch.int64)
    threads = torch.get_num_threads()

    def step():
        qd = torch.from_numpy(OQ.fake_quant_fp8_block(q_idx.numpy(), cfg.index_dim))
        sc = OA.indexer_scores(qd.unsqueeze(1), kd, w.unsqueeze(1), cfg.ratio, positions)
        idx = torch.from_numpy(OA.topk_indices(sc[:, 0], cfg.topk))
        toks = torch.arange(pos - cfg.window + 1, pos + 1) % cfg.window
        for r in range(cfg.batch):
            ents = torch.cat([win[r, toks], main[r, idx[r][idx[r] >= 0]]])
            OA.attend_entries(q[r], ents, sinks)

    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start < budget_s or len(times) < 2):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": cfg.batch / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"full config-2 decode step (32 rows: FP8 indexer over 8192 keys, top-2048, "
                      f"attention over 2176 entries x 128 heads), fp32 torch on dequantized caches, "
                      f"median of {len(times)} steps"}


def traffic_from_profiles(kernel: str):
    """HBM bytes per launch of `kernel` from the committed PMC summary, if one exists."""
    f = ROOT / "profiles" / "decode_step_c2_hbm_traffic.md"
    if not f.exists():
        return None
    m = re.search(rf"{kernel}\s+traffic_bytes_per_launch\s*=\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs are not part of it "
              f"(got --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_mib:
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4}))
        return
    nl = max(1, args.layers)
    built = [build_layer(torch, dev, args.nsplit, seed=1 + i) for i in range(nl)]
    layers = [b_[0] for b_ in built]
    inputs_all = [b_[1] for b_ in built]
    layer, inputs = layers[0], inputs_all[0]
    cfg = layer.cfg
    graph, _ = capture_layers(torch, layers, inputs_all)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed / (args.steps * nl) * 1e3  # per layer
    tokens_per_s = cfg.batch / (ms / 1e3)

    stages = stage_times(torch, layers, inputs_all, args.stage_iters or max(args.steps, 50))
    # algorithmic work per launch
    rows = cfg.batch
    entries = cfg.window + cfg.topk
    attn_bytes = rows * (entries * ENTRY_BYTES + QO_BYTES)
    attn_flops = rows * 4.0 * cfg.dim * cfg.heads * entries
    idx_bytes = rows * cfg.max_groups * IDX_KEY_BYTES
    idx_flops = rows * 2.0 * cfg.index_heads * cfg.index_dim * cfg.max_groups
    dominant = max(("sparse_mqa", "indexer_decode_fp8", "topk"), key=lambda k: stages[k])
    if dominant == "sparse_mqa":
        t = stages["sparse_mqa"] * 1e-6
        mfma_bound = attn_flops / (BF16_PEAK_TFLOPS * 1e12) > attn_bytes / (HBM_PEAK_GBS * 1e9)
        if mfma_bound:
            roof = {"bound": "mfma", "achieved": attn_flops / t / 1e12, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s"}
        else:
            roof = {"bound": "hbm", "achieved": attn_bytes / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    elif dominant == "indexer_decode_fp8":
        t = stages[dominant] * 1e-6
        roof = {"bound": "hbm", "achieved": idx_bytes / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    else:
        t = stages[dominant] * 1e-6
        sb = rows * cfg.max_groups * 4 + rows * cfg.topk * 4
        roof = {"bound": "hbm", "achieved": sb / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = traffic_from_profiles(dominant)
    roof["kernel"] = dominant
    roof["kernel_us"] = stages[dominant]

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, layer, inputs, args.cpu_seconds)

    out = {
        "metric": "decode tokens/s/GPU at 32k ctx (sparse MQA + indexer); % HBM/MFMA roofline",
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic (seeds 1..{nl}, one per layer), caches resident in HBM",
        "config": {"workload": "config2: decode B=32 ctx=32768, 128 heads x (512+64) FP8-b128 latent cache, "
                               "FP8 indexer 64x128 over 8192 groups (ratio 4), top-2048, window 128, sink",
                   "batch": cfg.batch, "context": 32768, "heads": cfg.heads, "latent": "512+64",
                   "index": "64x128 fp8", "topk": cfg.topk, "window": cfg.window, "nsplit": cfg.nsplit,
                   "graph_layers": nl, "step": "per attention layer, inside a graph replay of graph_layers layers"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "stages_us": stages,
        "step_roofline": {
            "hbm_bytes_alg": attn_bytes + idx_bytes,
            "ideal_us_hbm": (attn_bytes + idx_bytes) / (HBM_PEAK_GBS * 1e9) * 1e6,
            "frac_hbm": (attn_bytes + idx_bytes) / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9),
        },
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
