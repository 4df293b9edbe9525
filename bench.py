"""Decode throughput of the sparse-attention hot path on one MI355X.

Default workload (the headline metric): one CSA2 attention layer decoding
one token per row for B=32 rows at context 32768: bf16 queries, 128 heads over the shared
512+64 latent stored as FP8-b128 (656 B/entry), FP8 lightning indexer 64x128 over the 8192
compressed entries (ratio 4), top-2048, sliding window 128, per-head sink.  A "step" is one
replay of a HIP graph holding ``SparseDecodeLayer.step`` of --layers (default 8)
consecutive layers, each with its own caches and inputs, as a model's decode graph holds its
layers: per layer the group emission (the token's compressor projections into the carry
ring; every 4th token the group's pooling + norm, its rotated FP8-b128 cache entry and its
index key; the token's RoPE tables from the position table), the new token's kv RMSNorm +
RoPE + window append, the indexer query's RoPE + quantization and the indexer scores (one
launch), top-k, sparse MQA with the query's RoPE on load (split-KV), and the split merge with
the output's inverse RoPE and the positions' advance -- the per-token work of
``DeepseekV41Attention.forward`` between the projections.  At config 2 (8192 keys) the top-k
runs inside the attention launch (every attention workgroup of a row selects the row's list
from the scores itself); longer rows keep the top-k launch.  Every replay advances the positions, so the replays decode consecutive
tokens ending at position ctx-1 and emit a group every 4th step, as a decode loop does
(``--prologue rotated`` takes already-rotated q / q_idx / latent at a fixed position instead,
without emission, as the kernels' reference signatures do).  Distinct layers keep one layer's working set
(about 90 MB) from being served out of the last-level cache on the next step.  value =
B x layers / replay time (token-rows through one attention layer per second); ms_per_step
is per layer.  Inputs are synthetic and resident in HBM before timing starts.

--config 1 times the module drop-in (``mzoo_amd.owlet1.DeepseekV41Attention``) at BASELINE
config 1 -- one layer's forward over B=1, S=1024 (8 heads over 128+32, indexer 4x64, ratio 4,
top-128, window 64, fp32 weights ~N(0, 0.02), seed 0), value = tokens/s -- beside the CPU
oracle's module forward, and one module decode step at config-2 dimensions (B=32, context
32768, 128 heads over 512+64, indexer 64x128, top-2048, window 128, bf16) through the module's
cache layer.  --config 4 / 5 run the MXFP4-index decode (B=8, 32768 groups) and the hierarchical decode
(B=4: dense coarse branch of 4096 entries + MXFP4 fine index over 131072 groups) the same
way; --config 3 times the causal prefill (B=1, S=8192: FP8 indexer over 2048 groups ->
top-2048 -> sparse MQA with window 128 on every query row), value = query tokens/s.

Prints one JSON line (metric, value, roofline of the dominant kernel measured with HIP
events on its stream, cpu_baseline = the CPU oracle on this host's cores over a bounded
sample of the same workload).
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

# Algorithmic work (bytes a perfect kernel moves)
ENTRY_BYTES = 656                 # FP8-b128 latent entry
QO_BYTES = 2 * 128 * 576 * 2      # q read + out written per decoded row, bf16
KEY_BYTES = {"fp8": 132, "mxfp4": 68}  # indexer key: codes + scale(s)

METRIC = "decode tokens/s/GPU at 32k ctx (sparse MQA + indexer); % HBM/MFMA roofline"

DECODE = {
    2: dict(batch=32, ctx=32768, groups=8192, index_format="fp8", coarse_ratio=0, coarse_groups=0, nsplit=4, seed=1,
            text="config2: decode B=32 ctx=32768, 128 heads x (512+64) FP8-b128 latent cache, FP8 indexer 64x128 "
                 "over 8192 groups (ratio 4), top-2048, window 128, sink"),
    4: dict(batch=8, ctx=131072, groups=32768, index_format="mxfp4", coarse_ratio=0, coarse_groups=0, nsplit=14,
            seed=2, text="config4: decode B=8 ctx=131072, 128 heads x (512+64) FP8-b128 latent cache, MXFP4 indexer "
                         "64x128 over 32768 groups (ratio 4), top-2048, window 128, sink"),
    5: dict(batch=4, ctx=524288, groups=131072, index_format="mxfp4", coarse_ratio=128, coarse_groups=4096, nsplit=32,
            seed=4, text="config5: hierarchical decode B=4 ctx=524288, dense coarse branch of 4096 entries (ratio 128) "
                         "+ MXFP4 fine indexer 64x128 over 131072 groups, top-2048, window 128, merged by log-sum-exp"),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5], help="BASELINE configuration")
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--nsplit", type=int, default=0, help="attention splits per row (0: the config's default)")
    ap.add_argument("--layers", type=int, default=8, help="distinct attention layers in the replayed graph")
    ap.add_argument("--prologue", choices=["fused", "rotated"], default="fused",
                    help="fused: unrotated q / q_idx and the raw kv projection, norm and RoPE in the step's "
                         "launches; rotated: inputs already normed and rotated")
    ap.add_argument("--merge", choices=["inline", "launch"], default="launch",
                    help="split merge in the merge kernel, or inside the attention launch where it applies")
    ap.add_argument("--emit", choices=["merged", "separate"], default="merged",
                    help="group emission inside the indexer launch (merged) or in a launch of its own")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline time budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--stage-iters", type=int, default=0, help="launches per stage timing (0: max(steps, 50))")
    ap.add_argument("--kernels", action="store_true",
                    help="instead of the step: time the compressor and the quant / dequant kernels alone in "
                         "prefill shape (batch 1, seq 8192) and print their GB/s against 8 TB/s")
    ap.add_argument("--reindex", action="store_true",
                    help="instead of the step: time the two-level selection (dense scores + top-k, level one, "
                         "level two's candidate scorer + top-k) at growing cache lengths")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (3 launches): the reference kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    return ap.parse_args()


ROPE_THETA, COMPRESS_ROPE_THETA = 10000.0, 160000.0


def rope_inputs(torch, dev, positions):
    """bf16 cos / sin [B, 32] of the main and the compress RoPE at `positions` (the
    model-level position_embeddings and the indexer's tables)."""
    out = []
    for theta in (ROPE_THETA, COMPRESS_ROPE_THETA):
        inv = 1.0 / (theta ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
        f = torch.as_tensor(positions, dtype=torch.float32)[:, None] * inv
        out += [f.cos().bfloat16().to(dev), f.sin().bfloat16().to(dev)]
    return tuple(out)


def build_layer(torch, dev, nsplit=0, seed=None, config=2, fused=True, start=None, merged_emit=True):
    """A decode layer of BASELINE config `config` (2, 4 or 5) with synthetic history: the
    window ring holds the 128 tokens before the start position, every compressed group is
    published, and the first step decodes the token at `start` (default ctx-1).  With
    `fused` the layer holds a kv norm weight and the compressor weights of the in-step
    emission, and the inputs end with the token's fp32 compressor projections (the RoPE
    tables come from the layer's position table); otherwise they are pre-rotated."""
    from mzoo_amd.decode import CompressorWeights, DecodeConfig, SparseDecodeLayer
    c = DECODE[config]
    cfg = DecodeConfig(batch=c["batch"], heads=128, nope=512, rope=64, index_heads=64, index_dim=128, ratio=4,
                       window=128, topk=2048, max_groups=c["groups"], index_format=c["index_format"],
                       coarse_ratio=c["coarse_ratio"], coarse_groups=c["coarse_groups"], nsplit=nsplit or c["nsplit"],
                       merged_emit=merged_emit)
    ctx = c["ctx"]
    start = ctx - 1 if start is None else start
    gen = torch.Generator(device=dev).manual_seed(c["seed"] if seed is None else seed)
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev)  # noqa: E731
    sinks = rnd(cfg.heads)
    kv_w = (1.0 + 0.1 * rnd(cfg.dim)).bfloat16() if fused else None
    cw = None
    if fused:
        cw = CompressorWeights(norm_weight=(1.0 + 0.1 * rnd(cfg.dim)).bfloat16(),
                               wk=(0.04 * rnd(cfg.index_dim, cfg.dim)).bfloat16(),
                               k_norm_weight=(1.0 + 0.1 * rnd(cfg.index_dim)).bfloat16(),
                               coarse_norm_weight=(1.0 + 0.1 * rnd(cfg.dim)).bfloat16() if cfg.coarse_ratio else None,
                               rope_theta=COMPRESS_ROPE_THETA)
    layer = SparseDecodeLayer(cfg, dev, sinks=sinks, kv_norm_weight=kv_w, compressor=cw, max_position=ctx)
    b, d = cfg.batch, cfg.dim
    layer.fill_window(rnd(b, cfg.window, d).bfloat16(), start - 1)
    # groups in chunks (bounds the staging buffers of the larger configs)
    step = max(1, (1 << 27) // (b * d))
    for g0 in range(0, cfg.max_groups, step):
        n = min(step, cfg.max_groups - g0)
        layer.append_groups(g0, rnd(b, n, d).bfloat16(), rnd(b, n, cfg.index_dim).bfloat16())
    if cfg.coarse_ratio:
        layer.fill_coarse(rnd(b, cfg.coarse_groups, d).bfloat16())
    layer.set_positions(start)
    q = rnd(b, cfg.heads, d).bfloat16()
    kv = rnd(b, d).bfloat16()
    q_idx = rnd(b, cfg.index_heads, cfg.index_dim).bfloat16()
    w = rnd(b, cfg.index_heads) * cfg.index_heads ** -0.5
    extra = ()
    if fused:
        # the carried partial group and the token's compressor projections
        layer.set_carry(rnd(b, start % cfg.ratio, d), rnd(b, start % cfg.ratio, d))
        extra = (rnd(b, d), rnd(b, d))
        if cfg.coarse_ratio:
            layer.set_carry(rnd(b, start % cfg.coarse_ratio, d), rnd(b, start % cfg.coarse_ratio, d), coarse=True)
            extra += (rnd(b, d), rnd(b, d))
    return layer, (q, kv, q_idx, w) + extra, sinks


def run_step(layer, inp, advance=False):
    """``SparseDecodeLayer.step`` on bench inputs: with compressor projections (the fused
    step) the emission runs first and the RoPE tables come from the position table."""
    if len(inp) > 4:
        return layer.step(*inp[:4], rope="table", compress=inp[4:], advance=advance)
    return layer.step(*inp[:4])


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
                run_step(layer, st)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for layer, st in zip(layers, statics):
            run_step(layer, st, advance=len(st) > 4)
    return g, statics


def graph_time(torch, fns, iters):
    """Average duration of one launch among `fns` (called in turn): a HIP graph of at least
    32 back-to-back launches, replayed and timed with HIP events on the stream the kernels
    run on.  Inside a graph the launches follow each other with no host gap, so the figure
    is the kernels' own duration."""
    n = len(fns)
    reps = max(1, (32 + n - 1) // n)
    replays = max(1, iters // (reps * n))
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
    return time_launches(torch, g.replay, replays) / (reps * n)


def stage_times(torch, layers, inputs, iters):
    """Average duration of each kernel of the step alone, launch after launch cycling
    through the layers (consecutive launches read different caches, as in the decode graph).
    The emission is timed at three positions -- one that completes a group of every branch,
    one that completes a fine group only (configs with a coarse branch) and one that only
    carries the token -- and amortized over the branches' ratios (1 of `ratio` steps completes
    a fine group, 1 of `coarse_ratio` a coarse one)."""
    per_layer = [stage_fns(torch, layer, inp) for layer, inp in zip(layers, inputs)]
    # the launches whose work depends on the position: the emission, or the merged emission +
    # scores launch
    moving = [k for k in per_layer[0] if k.startswith(("decode_emit", "indexer_emit"))]
    timed = {k: [d.pop(k) for d in per_layer] for k in moving}
    out = {name: graph_time(torch, [d[name] for d in per_layer], iters) for name in per_layer[0]}
    for key, fns in timed.items():
        cfg = layers[0].cfg
        saved = [int(layer.positions[0]) for layer in layers]
        period = cfg.ratio * max(cfg.coarse_ratio // cfg.ratio, 1) if cfg.coarse_ratio else cfg.ratio
        p_all = (saved[0] + 1) // period * period - 1  # completes every branch's group
        if p_all < period:
            p_all += period

        def at(pos):
            for layer in layers:
                layer.set_positions(pos)
            return graph_time(torch, fns, iters)
        out[key + "_group"] = at(p_all)
        out[key + "_carry"] = at(p_all - 1)
        amort = (out[key + "_group"] + (cfg.ratio - 1) * out[key + "_carry"]) / cfg.ratio
        if cfg.coarse_ratio:
            out[key + "_fine_group"] = at(p_all - cfg.ratio)
            n_fine = cfg.coarse_ratio // cfg.ratio
            amort = (out[key + "_group"] + (n_fine - 1) * out[key + "_fine_group"] +
                     (cfg.coarse_ratio - n_fine) * out[key + "_carry"]) / cfg.coarse_ratio
        out[key] = amort
        for layer, p in zip(layers, saved):
            layer.set_positions(p)
    return out


def stage_fns(torch, layer, inputs):
    """The step's launches for one layer, each callable alone."""
    from mzoo_amd import _lib, indexer
    from mzoo_amd import csa2_attn as MA
    cfg = layer.cfg
    b = cfg.batch
    q, kv, q_idx, w = inputs[:4]
    emit = len(inputs) > 4
    rope = (layer.step_cos, layer.step_sin, layer.step_cos, layer.step_sin) if emit else ()
    ws = layer.workspace
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    fns = {}
    fp8 = cfg.index_format == "fp8"
    pro = emit and layer._emit_prologue
    merged = pro and layer._merged_emit
    if merged:
        # the emission and the scores in one launch (window entry and query prologue included)
        fns["indexer_emit_fp8" if fp8 else "indexer_emit_mxfp4"] = \
            lambda: layer._emit_scores(inputs[4:], kv, q_idx, w)
    elif emit:
        # the in-step group emission (one launch per compressed branch); the first launch also
        # runs the step's prologue (window entry, indexer query RoPE + quantization)
        fns["decode_emit"] = lambda: layer._emit(inputs[4:], True, prologue=(kv, q_idx) if pro else None)
    pos = layer.positions.view(b, 1)
    if merged:
        pass
    elif pro:
        # the plain scorer over the quantized query
        if fp8:
            fns["indexer_scores_fp8"] = lambda: indexer.scores_fp8(
                layer.q_codes, layer.q_scales, w.view(b, 1, -1), layer.k_codes, layer.k_scales,
                compress_ratio=cfg.ratio, positions=pos, out=layer.scores)
        else:
            fns["indexer_scores_mxfp4"] = lambda: indexer.scores_mxfp4(
                layer.q_codes, layer.q_e8m0, w.view(b, 1, -1), layer.k_packed, layer.k_e8m0,
                compress_ratio=cfg.ratio, positions=pos, out=layer.scores)
    elif rope:
        cos, sin, icos, isin = rope

        def indexer_fused():
            # kv RMSNorm + RoPE + window append, query RoPE + quantization, scores: one launch
            _lib.call("mzk_indexer_decode_fused", 0 if fp8 else 1, q_idx.data_ptr(), w.data_ptr(),
                      (layer.k_codes if fp8 else layer.k_packed).data_ptr(),
                      (layer.k_scales if fp8 else layer.k_e8m0).data_ptr(), b, cfg.index_heads, cfg.index_dim,
                      cfg.max_groups, cfg.max_groups, layer.positions.data_ptr(), cfg.ratio, layer.scores.data_ptr(),
                      cfg.max_groups, None, None, icos.data_ptr(), isin.data_ptr(), 64, kv.data_ptr(),
                      layer.kv_norm_weight.data_ptr(), layer.kv_norm_eps, cos.data_ptr(), sin.data_ptr(), cfg.nope,
                      cfg.rope, layer.win.data_ptr(), cfg.window, cfg.window, st())
        fns["indexer_decode_fp8" if fp8 else "indexer_decode_mxfp4"] = indexer_fused
    elif fp8:
        def indexer_decode():
            # window append + indexer-query quantization + FP8 scores: the step's first launch
            _lib.call("mzk_indexer_decode_fp8", q_idx.data_ptr(), w.data_ptr(), layer.k_codes.data_ptr(),
                      layer.k_scales.data_ptr(), b, cfg.index_heads, cfg.index_dim, cfg.max_groups, cfg.max_groups,
                      layer.positions.data_ptr(), cfg.ratio, layer.scores.data_ptr(), cfg.max_groups, None, None,
                      kv.data_ptr(), cfg.nope, cfg.rope, layer.win.data_ptr(), cfg.window, cfg.window, st())
        fns["indexer_decode_fp8"] = indexer_decode
    else:
        def indexer_decode():
            # window append + indexer-query MXFP4 quantization + scores: one launch
            _lib.call("mzk_indexer_decode_mxfp4", q_idx.data_ptr(), w.data_ptr(), layer.k_packed.data_ptr(),
                      layer.k_e8m0.data_ptr(), b, cfg.index_heads, cfg.index_dim, cfg.max_groups, cfg.max_groups,
                      layer.positions.data_ptr(), cfg.ratio, layer.scores.data_ptr(), cfg.max_groups, None, None,
                      kv.data_ptr(), cfg.nope, cfg.rope, layer.win.data_ptr(), cfg.window, cfg.window, st())
        fns["indexer_decode_mxfp4"] = indexer_decode
    fns["topk"] = lambda: indexer.topk(layer.scores.view(b, cfg.max_groups), cfg.topk, out=layer.idx,
                                       workspace=layer.topk_ws)
    coarse = layer.coarse
    # the decode graph, replayed before the stages are timed, counted its in-launch merges in
    # the workspace: then the attention launch is timed with its merge and nothing follows it
    inline = MA.merge_status(ws, b, cfg.heads, cfg.dim, cfg.nsplit + layer.nsplit_wd)[1] > 0

    def attn():
        # the split-KV attention kernel alone: with no `out` the entry point writes the
        # split partials into the workspace and launches nothing else; with the in-launch
        # merge the launch also merges them into `out`
        args = (q.data_ptr(), b, 1, cfg.heads, cfg.dim, 1, cfg.nope, layer.positions.data_ptr(),
                layer.win.data_ptr(), cfg.window, cfg.window, cfg.window,
                None if coarse is None else coarse.data_ptr(), cfg.coarse_groups, cfg.coarse_groups,
                max(cfg.coarse_ratio, 1), layer.main.data_ptr(), cfg.max_groups, cfg.max_groups,
                layer.idx.data_ptr(), cfg.topk, cfg.topk, layer.sinks.data_ptr(), cfg.nsplit, ws.data_ptr(),
                ws.numel() * ws.element_size(), *((layer.out.data_ptr(), layer.lse.data_ptr()) if inline else
                                                  (None, None)))
        if rope:
            _lib.call("mzk_sparse_mqa_rope", *args, rope[0].data_ptr(), rope[1].data_ptr(), cfg.rope, st())
        else:
            _lib.call("mzk_sparse_mqa", *args, st())
    fns["sparse_mqa"] = attn
    if layer.selects_in_attention:
        # the step's attention launch: the row's top-k selected inside it from the scores (the
        # "topk" and "sparse_mqa" stages above are the two launches it replaces)
        def attn_select():
            _lib.call("mzk_sparse_mqa_select", q.data_ptr(), b, cfg.heads, cfg.dim, 1, cfg.nope,
                      layer.positions.data_ptr(), 0, layer.win.data_ptr(), cfg.window, cfg.window, cfg.window,
                      None if coarse is None else coarse.data_ptr(), cfg.coarse_groups, cfg.coarse_groups,
                      max(cfg.coarse_ratio, 1), layer.main.data_ptr(), cfg.max_groups, cfg.max_groups,
                      layer.scores.data_ptr(), cfg.max_groups, cfg.topk, layer.idx.data_ptr(), cfg.topk,
                      layer.sinks.data_ptr(), cfg.nsplit, ws.data_ptr(), ws.numel() * ws.element_size(),
                      *((layer.out.data_ptr(), layer.lse.data_ptr()) if inline else (None, None)),
                      *((rope[0].data_ptr(), rope[1].data_ptr(), cfg.rope) if rope else (None, None, 0)), st())
        fns["sparse_mqa_select"] = attn_select
    if inline:
        pass
    elif rope:
        fns["sparse_mqa_combine"] = lambda: _lib.call(
            "mzk_sparse_mqa_combine_rope", ws.data_ptr(), b, 1, cfg.heads, cfg.dim, cfg.nsplit,
            layer.sinks.data_ptr(), rope[0].data_ptr(), rope[1].data_ptr(), cfg.rope, layer.out.data_ptr(),
            layer.lse.data_ptr(), st())
    else:
        fns["sparse_mqa_combine"] = lambda: _lib.call(
            "mzk_sparse_mqa_combine", ws.data_ptr(), b, 1, cfg.heads, cfg.dim, cfg.nsplit, layer.sinks.data_ptr(),
            layer.out.data_ptr(), layer.lse.data_ptr(), st())
    return fns


def cpu_baseline(torch, layer, inputs, budget_s, rows=None):
    """The CPU oracle's decode step (indexer scores -> top-k -> attention over window
    [+ coarse] + selected entries) in fp32 on the dequantized caches, for `rows` (default
    all) of the batch, on this host's cores; median of repeated steps."""
    import numpy as np

    from mzoo_amd import quant
    from oracle import attention as OA
    from oracle import compressor as OC
    from oracle import quant as OQ
    cfg = layer.cfg
    rows = list(range(cfg.batch)) if rows is None else rows
    q, kv, q_idx, w = (t.float().cpu()[rows] for t in inputs[:4])
    emit = len(inputs) > 4
    tabs = []
    if emit:
        # the step's RoPE tables: row `pos` of the layer's position table (main and indexer)
        p_ = int(layer.positions[0])
        row = layer.rope_table[p_].float().cpu().numpy()
        c_, s_ = (np.repeat(row[None, :32], len(rows), 0), np.repeat(row[None, 32:], len(rows), 0))
        tabs = [c_, s_, c_, s_]
        cw = layer.compressor
        e_nw, e_wk, e_kw = (t.float().cpu().numpy() for t in (cw.norm_weight, cw.wk, cw.k_norm_weight))
        e_kv = np.random.default_rng(0).standard_normal((len(rows), cfg.ratio, cfg.dim)).astype(np.float32)
    kv_w = None if layer.kv_norm_weight is None else layer.kv_norm_weight.float().cpu().numpy()
    win = quant.unpack_latent_fp8_b128(layer.win[rows], dtype=torch.float32).cpu()
    main = quant.unpack_latent_fp8_b128(layer.main[rows], dtype=torch.float32).cpu()
    coarse = None
    if layer.coarse is not None:
        coarse = quant.unpack_latent_fp8_b128(layer.coarse[rows], dtype=torch.float32).cpu()
    if cfg.index_format == "fp8":
        kd = layer.k_codes[rows].cpu().view(torch.float8_e4m3fn).float() * layer.k_scales[rows].cpu().unsqueeze(-1)
    else:
        kd = quant.dequant_mxfp4(layer.k_packed[rows], layer.k_e8m0[rows]).cpu()
    sinks = layer.sinks.cpu()
    pos = int(layer.positions[0])
    positions = torch.full((len(rows), 1), pos, dtype=torch.int64)
    nc = 0 if coarse is None else min(cfg.coarse_groups, (pos + 1) // cfg.coarse_ratio)
    threads = torch.get_num_threads()

    def step():
        qx, qi = q, q_idx
        if emit:
            # the group emission, amortized: one row in `ratio` completes a group per step
            n_emit = max(1, -(-len(rows) // cfg.ratio))
            OC.emit_group(e_kv[:n_emit], e_kv[:n_emit], cfg.ratio, e_nw, cw.eps, tabs[0][:n_emit], tabs[1][:n_emit],
                          e_wk, e_kw, cw.k_eps)
        if tabs:
            # the fused prologue: query / indexer-query RoPE, the new latent's norm + RoPE + packing
            cos, sin, icos, isin = tabs
            qx = torch.from_numpy(OC.rope(q.numpy(), cos[:, None], sin[:, None], dtype="bfloat16"))
            qi = torch.from_numpy(OC.rope(q_idx.numpy(), icos[:, None], isin[:, None], dtype="bfloat16"))
            OQ.pack_latent_fp8_b128(OC.decode_kv_latent(kv.numpy(), kv_w, layer.kv_norm_eps, cos, sin))
        if cfg.index_format == "fp8":
            qd = torch.from_numpy(OQ.fake_quant_fp8_block(qi.numpy(), cfg.index_dim))
        else:
            qd = torch.from_numpy(OQ.fake_quant_fp4_block(qi.numpy(), 32))
        sc = OA.indexer_scores(qd.unsqueeze(1), kd, w.unsqueeze(1), cfg.ratio, positions)
        idx = torch.from_numpy(OA.topk_indices(sc[:, 0], cfg.topk))
        toks = torch.arange(pos - cfg.window + 1, pos + 1) % cfg.window
        for i in range(len(rows)):
            parts = [win[i, toks]] + ([coarse[i, :nc]] if coarse is not None else [])
            ents = torch.cat(parts + [main[i, idx[i][idx[i] >= 0]]])
            o = OA.attend_entries(qx[i], ents, sinks)[0]
            if tabs:
                OC.rope(o.numpy(), tabs[0][i], tabs[1][i], inverse=True, dtype="bfloat16")

    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start < budget_s or len(times) < 2):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    entries = cfg.window + nc + cfg.topk
    return {"value": len(rows) / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"decode step of {len(rows)} of {cfg.batch} rows ("
                      f"{'group emission for 1 row in ' + str(cfg.ratio) + ', ' if emit else ''}"
                      f"{'kv norm + RoPE, q / q_idx RoPE, ' if tabs else ''}{cfg.index_format} indexer over "
                      f"{cfg.max_groups} keys, top-{cfg.topk}, attention over {entries} entries x {cfg.heads} heads), "
                      f"fp32 torch on dequantized caches, median of {len(times)} steps"}


def traffic_from_profiles(kernel: str, config: int):
    """HBM bytes per launch of `kernel` from the committed PMC summary, if one exists."""
    f = ROOT / "profiles" / f"decode_step_c{config}_hbm_traffic.md"
    if not f.exists():
        return None
    m = re.search(rf"{kernel}\s+traffic_bytes_per_launch\s*=\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def roofline(kind, flops, nbytes, t_us, peak_tflops=BF16_PEAK_TFLOPS):
    """The binding roof of one kernel: MFMA if its ideal compute time exceeds its ideal
    HBM time (or kind == "mfma"), else HBM; achieved = algorithmic work / measured duration."""
    t = t_us * 1e-6
    if kind == "mfma" or (kind is None and flops / (peak_tflops * 1e12) > nbytes / (HBM_PEAK_GBS * 1e9)):
        r = {"bound": "mfma", "achieved": flops / t / 1e12, "peak": peak_tflops, "unit": "TFLOP/s"}
    else:
        r = {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    r["frac"] = r["achieved"] / r["peak"]
    return r


def run_decode(torch, dev, args):
    c = DECODE[args.config]
    nl = max(1, args.layers)
    fused = args.prologue == "fused"
    # the replays advance the positions: the last timed replay decodes position ctx-1
    start = c["ctx"] - 1 - (args.warmup + args.steps) if fused else None
    built = [build_layer(torch, dev, args.nsplit, seed=c["seed"] + i, config=args.config, fused=fused,
                         merged_emit=args.emit == "merged",
                         start=start) for i in range(nl)]
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
    pos = c["ctx"] - 1
    nc = min(cfg.coarse_groups, (pos + 1) // cfg.coarse_ratio) if cfg.coarse_ratio else 0
    entries = cfg.window + nc + cfg.topk
    attn_bytes = rows * (entries * ENTRY_BYTES + QO_BYTES)
    attn_flops = rows * 4.0 * cfg.dim * cfg.heads * entries
    idx_bytes = rows * cfg.max_groups * KEY_BYTES[cfg.index_format]
    idx_flops = rows * 2.0 * cfg.index_heads * cfg.index_dim * cfg.max_groups
    idx_stage = next(k for k in ("indexer_emit_fp8", "indexer_emit_mxfp4", "indexer_scores_fp8",
                                 "indexer_scores_mxfp4", "indexer_decode_fp8", "indexer_decode_mxfp4") if k in stages)
    # the dominant single kernel among the step's launches: with the top-k inside the
    # attention launch that launch (it also reads the scores and writes the list); else the
    # attention and the top-k launch -- rows longer than 32768 keys run the top-k as three
    # launches (a latency stage, not one kernel), so it is a candidate only as one launch
    if "sparse_mqa_select" in stages:
        cands = ("sparse_mqa_select", idx_stage)
    else:
        cands = ("sparse_mqa", idx_stage) + (("topk",) if cfg.max_groups <= 32768 else ())
    dominant = max(cands, key=lambda k: stages[k])
    if dominant == "sparse_mqa_select":
        roof = roofline(None, attn_flops, attn_bytes + rows * (cfg.max_groups + cfg.topk) * 4, stages[dominant])
    elif dominant == "sparse_mqa":
        roof = roofline(None, attn_flops, attn_bytes, stages[dominant])
    elif dominant == idx_stage:
        roof = roofline("hbm", idx_flops, idx_bytes, stages[dominant])
    else:
        roof = roofline("hbm", 0.0, rows * cfg.max_groups * 4 + rows * cfg.topk * 4, stages[dominant])
    roof["traffic"] = traffic_from_profiles(dominant, args.config)
    roof["kernel"] = dominant
    roof["kernel_us"] = stages[dominant]

    cpu = None
    if not args.no_cpu:
        # at most 2^18 (row, key) pairs of indexer work on the CPU: all 32 rows of config 2
        cpu_rows = None if rows * cfg.max_groups <= (1 << 18) else list(range(max(1, (1 << 18) // cfg.max_groups)))
        cpu = cpu_baseline(torch, layer, inputs, args.cpu_seconds, rows=cpu_rows)

    return {
        "metric": METRIC,
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
        "data": f"synthetic (seeds {c['seed']}..{c['seed'] + nl - 1}, one per layer), caches resident in HBM",
        "config": {"workload": c["text"], "batch": cfg.batch, "context": c["ctx"], "heads": cfg.heads,
                   "latent": "512+64", "index": f"64x128 {cfg.index_format}", "topk": cfg.topk,
                   "window": cfg.window, "coarse": nc, "nsplit": cfg.nsplit, "graph_layers": nl,
                   "split_merge": "merge kernel" if "sparse_mqa_combine" in stages else "inside the attention launch",
                   "emission": ("inside the indexer launch" if layer._merged_emit else "launch of its own")
                   if fused else None,
                   "selection": "inside the attention launch" if layer.selects_in_attention else "top-k launch",
                   "step": "per attention layer, inside a graph replay of graph_layers layers",
                   "prologue": ("fused: in-step group emission (carry ring, pooling + norm, cache entry and "
                                "index key every 4th token; RoPE tables from the position table), kv RMSNorm + "
                                "RoPE + window append, q / q_idx RoPE and the output's inverse RoPE inside the "
                                "step's launches; positions advance every replay") if fused else
                               "rotated: q, q_idx and the new latent arrive normed and rotated"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "stages_us": stages,
        "step_roofline": {
            "hbm_bytes_alg": attn_bytes + idx_bytes,
            "ideal_us_hbm": (attn_bytes + idx_bytes) / (HBM_PEAK_GBS * 1e9) * 1e6,
            "frac_hbm": (attn_bytes + idx_bytes) / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9),
        },
    }


def run_prefill(torch, dev, args):
    """causal prefill B=1, S=8192, 128 heads over 512+64 (bf16 latent),
    FP8 indexer 64x128 over 2048 groups (ratio 4), top-2048, window 128, sink.  One step =
    indexer-query quantization -> FP8 scores -> top-k -> sparse MQA over all query rows."""
    from mzoo_amd import csa2_attn, indexer, quant
    b, s, h, d, g, k, win, ratio, hi, di = 1, 8192, 128, 576, 2048, 2048, 128, 4, 64, 128
    gen = torch.Generator(device=dev).manual_seed(3)
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev)  # noqa: E731
    q = rnd(b, s, h, d).bfloat16()
    kv = rnd(b, s, 1, d).bfloat16()
    main = rnd(b, g, 1, d).bfloat16()
    q_idx = rnd(b, s, hi, di).bfloat16()
    k_idx = rnd(b, g, di).bfloat16()
    w = rnd(b, s, hi) * hi ** -0.5
    sinks = rnd(h)
    kc, ks = quant.quant_fp8_block(k_idx, 128)  # the published key cache
    ks = ks[..., 0].contiguous()
    scores = torch.empty(b, s, g, dtype=torch.float32, device=dev)
    idx = torch.empty(b, s, k, dtype=torch.int32, device=dev)
    state = {}

    def quant_q():
        qc, qs = quant.quant_fp8_block(q_idx, 128)
        state["q"] = (qc, qs[..., 0].contiguous())

    def scores_fp8():
        qc, qs = state["q"]
        indexer.scores_fp8(qc, qs, w, kc, ks, compress_ratio=ratio, out=scores)

    def topk():
        indexer.topk(scores, k, out=idx)

    def attn():
        state["o"] = csa2_attn.fwd(q, kv, main, idx, window=win, compress_ratio=ratio, sinks=sinks)

    def step():
        quant_q()
        scores_fp8()
        topk()
        attn()

    steps = min(args.steps, 20)
    warm = min(args.warmup, 3) + 1
    for _ in range(warm):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    # each stage alone, as a graph of back-to-back launches (the kernels' own time, without
    # the host's launch gaps, which exceed the shorter kernels)
    stages = {"quant_q": graph_time(torch, [quant_q], 64), "indexer_fp8": graph_time(torch, [scores_fp8], 64),
              "topk": graph_time(torch, [topk], 64), "sparse_mqa": graph_time(torch, [attn], 32)}
    t = torch.arange(s, dtype=torch.float64)
    pairs = float((torch.clamp((t + 1) // ratio, max=k) + torch.clamp(t + 1, max=win)).sum())
    attn_flops = 4.0 * d * h * pairs
    attn_bytes = 2.0 * s * h * d * 2 + (s * d + g * d) * 2 + s * k * 4
    vis = float(torch.clamp((t + 1) // ratio, max=g).sum())
    idx_flops = 2.0 * hi * di * vis
    dominant = max(("sparse_mqa", "indexer_fp8", "topk"), key=lambda x: stages[x])
    if dominant == "sparse_mqa":
        roof = roofline("mfma", attn_flops, attn_bytes, stages[dominant])
    elif dominant == "indexer_fp8":
        roof = roofline("mfma", idx_flops, s * hi * di + g * 132, stages[dominant], FP8_PEAK_TFLOPS)
    else:
        roof = roofline("hbm", 0.0, s * g * 4 + s * k * 4, stages[dominant])
    roof["traffic"] = None
    roof["kernel"] = dominant
    roof["kernel_us"] = stages[dominant]

    cpu = None
    if not args.no_cpu:
        cpu = prefill_cpu_baseline(torch, q, kv, main, q_idx, k_idx, w, sinks, win, ratio, k, args.cpu_seconds)
    return {
        "metric": METRIC,
        "value": s / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seed 3), resident in HBM",
        "config": {"workload": "config3: causal prefill B=1 S=8192, 128 heads x (512+64) bf16 latent, FP8 indexer "
                               "64x128 over 2048 groups (ratio 4), top-2048, window 128, sink",
                   "batch": b, "seq_len": s, "heads": h, "topk": k, "window": win,
                   "step": "whole prefill (query quantization, FP8 scores, top-k, sparse MQA)"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "stages_us": stages,
    }


def prefill_cpu_baseline(torch, q, kv, main, q_idx, k_idx, w, sinks, win, ratio, k, budget_s):
    """The oracle's prefill on 16 query rows spread evenly over the sequence."""
    from oracle import attention as OA
    from oracle import quant as OQ
    s = q.shape[1]
    rows = list(range(s - 1, -1, -(s // 16)))[:16]
    qd = torch.from_numpy(OQ.fake_quant_fp8_block(q_idx[:, rows].float().cpu().numpy(), 128))
    kd = torch.from_numpy(OQ.fake_quant_fp8_block(k_idx.float().cpu().numpy(), 128))
    wr = w[:, rows].cpu()
    qr = q[0, rows].float().cpu()
    kvc, mainc, sk = kv[0, :, 0].float().cpu(), main[0, :, 0].float().cpu(), sinks.cpu()
    pos = torch.tensor(rows, dtype=torch.int64).view(1, -1)

    def step():
        sc = OA.indexer_scores(qd, kd, wr, ratio, pos)
        idx = OA.topk_indices(sc[0], k)
        for i, t in enumerate(rows):
            sel = torch.from_numpy(idx[i][idx[i] >= 0])
            OA.attend_entries(qr[i], torch.cat([kvc[max(0, t - win + 1):t + 1], mainc[sel]]), sk)

    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start < budget_s or len(times) < 2):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": len(rows) / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(rows)} query rows of the 8192-row prefill (FP8 indexer over 2048 keys, top-2048, "
                      f"attention over window + selected entries x 128 heads), fp32 torch, median of {len(times)} runs"}


def run_kernels(torch, dev, args):
    """The compressor and the quant / dequant kernels alone, in the prefill shape of BASELINE
    config 3 (batch 1, seq 8192, latent 512 + 64, indexer 64 x 128, ratio 4): each launch
    timed in a graph of back-to-back launches (HIP events on the launch stream), bytes =
    the kernel's algorithmic reads + writes."""
    from mzoo_amd import cache, quant
    t, d, hi, di, r = 8192, 576, 64, 128, 4
    gen = torch.Generator(device=dev).manual_seed(3)
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev)  # noqa: E731
    kv, gate = rnd(1, t, d), rnd(1, t, d)
    nw = (1.0 + 0.1 * rnd(d)).bfloat16()
    out_lat = torch.empty(1, t // r, d, dtype=torch.bfloat16, device=dev)
    q = rnd(t, hi, di).bfloat16()
    x = rnd(t, d).bfloat16()
    ent = quant.pack_latent_fp8_b128(x)
    codes, scales = quant.quant_fp8_block(q, 128)
    packed, e8 = quant.quant_mxfp4(q)
    iters = max(args.stage_iters, 200)
    eb = quant.entry_bytes()
    cases = {
        # the compressor: fp32 kv + gate of 8192 tokens -> 2048 normed bf16 groups
        "compress_r4": (lambda: cache.compress(kv, gate, r, nw, 1e-6, torch.bfloat16, out=out_lat),
                        2 * t * d * 4 + (t // r) * d * 2 + d * 2),
        # the indexer query quantizers: bf16 [8192 x 64 x 128] -> FP8 b128 / MXFP4
        "quant_fp8_b128": (lambda: quant.quant_fp8_block(q, 128), t * hi * di * 2 + t * hi * di + t * hi * 4),
        "quant_mxfp4": (lambda: quant.quant_mxfp4(q), t * hi * di * 2 + t * hi * di // 2 + t * hi * di // 32),
        "dequant_fp8_b128": (lambda: quant.dequant_fp8_block(codes, scales, 128, dtype=torch.bfloat16),
                             t * hi * di + t * hi * 4 + t * hi * di * 2),
        "dequant_mxfp4": (lambda: quant.dequant_mxfp4(packed, e8, dtype=torch.bfloat16),
                          t * hi * di // 2 + t * hi * di // 32 + t * hi * di * 2),
        # the latent cache entries: bf16 [8192 x 576] <-> 656-byte FP8-b128 entries
        "pack_latent_fp8_b128": (lambda: quant.pack_latent_fp8_b128(x, out=ent), t * d * 2 + t * eb),
        "unpack_latent_fp8_b128": (lambda: quant.unpack_latent_fp8_b128(ent), t * eb + t * d * 2),
    }
    res = {}
    for name, (fn, nbytes) in cases.items():
        us = graph_time(torch, [fn], iters)
        res[name] = {"us": round(us, 3), "bytes": int(nbytes), "GB/s": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
    return {"metric": "prefill-shape kernel bandwidth", "unit": "GB/s", "peak": HBM_PEAK_GBS,
            "config": {"workload": "config3 prefill shape: batch 1, seq 8192, latent 512+64, indexer 64x128, "
                                   "ratio 4", "iters": iters}, "kernels": res}


def run_reindex(torch, dev, args):
    """The two-level selection's cost against the cache length T (tickets/0009: level two
    is O(candidates), not O(T)).  Per T, batch rows at their last position, MXFP4 (B=4, the
    config-5 indexer) and FP8 (B=32, the config-2 indexer) keys: the dense score kernel and
    its top-2048 (what a layer without candidates pays), level one's block selection (the
    candidate source's extra work), and level two -- the candidate scorer over 2048 blocks
    of 8 plus its top-2048 mapped to key positions.  Each launch timed in a graph of
    back-to-back launches (HIP events on the launch stream)."""
    from mzoo_amd import indexer as MI
    from mzoo_amd import quant
    nblk, bs, k, hi, di, ratio = 2048, 8, 2048, 64, 128, 4
    iters = max(args.stage_iters, 200)
    out = {}
    for fmt, b in (("mxfp4", 4), ("fp8", 32)):
        for t in (16384, 65536, 131072, 262144):
            gen = torch.Generator(device=dev).manual_seed(t + b)
            q = torch.randn(b, 1, hi, di, generator=gen, device=dev).bfloat16()
            kk = torch.randn(b, t, di, generator=gen, device=dev).bfloat16()
            w = torch.randn(b, 1, hi, generator=gen, device=dev) * hi ** -0.5
            pos = torch.full((b, 1), t * ratio - 1, dtype=torch.int64, device=dev)
            lens = torch.full((b, 1, 1), t, dtype=torch.int64, device=dev)
            if fmt == "mxfp4":
                qa, qb = quant.quant_mxfp4(q)
                ka, kb = quant.quant_mxfp4(kk)
                dense_fn, cand_fn = MI.scores_mxfp4, MI.candidate_scores_mxfp4
            else:
                qa, qs = quant.quant_fp8_block(q, 128)
                ka, ks = quant.quant_fp8_block(kk, 128)
                qb, kb = qs[..., 0].contiguous(), ks[..., 0].contiguous()
                dense_fn, cand_fn = MI.scores_fp8, MI.candidate_scores_fp8
            del kk
            dense = torch.empty(b, 1, t, dtype=torch.float32, device=dev)
            cs = torch.empty(b, 1, nblk * bs, dtype=torch.float32, device=dev)
            idx = torch.empty(b, 1, k, dtype=torch.int32, device=dev)
            cidx = torch.empty(b, 1, k, dtype=torch.int32, device=dev)
            ws = torch.empty(max(MI.topk_workspace_bytes(b, t), MI.topk_workspace_bytes(b, nblk * bs), 16),
                             dtype=torch.uint8, device=dev)
            dense_fn(qa, qb, w, ka, kb, compress_ratio=ratio, positions=pos, out=dense)
            cand = MI.candidate_block_list(dense, lens, nblk, bs)
            fns = {
                "dense_scores": lambda: dense_fn(qa, qb, w, ka, kb, compress_ratio=ratio, positions=pos, out=dense),
                "dense_topk": lambda: MI.topk(dense, k, out=idx, workspace=ws),
                "level1_select": lambda: MI.candidate_block_list(dense, lens, nblk, bs, out=cand),
                "level2_scores": lambda: cand_fn(qa, qb, w, ka, kb, cand, block_size=bs, compress_ratio=ratio,
                                                 positions=pos, out=cs),
                "level2_topk": lambda: MI.candidate_topk(cs, cand, bs, k, out=cidx, workspace=ws),
            }
            row = {name: round(graph_time(torch, [fn], iters), 3) for name, fn in fns.items()}
            kb_bytes = (di // 2 + di // 32) if fmt == "mxfp4" else di + 4
            row["level2_score_GB/s"] = round(b * nblk * bs * (kb_bytes + 4) / row["level2_scores"] / 1e3, 1)
            out[f"{fmt}_B{b}_T{t}"] = row
            print(f"reindex {fmt} B={b} T={t}: {row}", file=sys.stderr, flush=True)
            del qa, qb, ka, kb, dense, cs
    return {"metric": "two-level selection cost vs cache length", "unit": "us per launch",
            "config": {"workload": "decode rows at their last position; 2048 candidate blocks of 8, top-2048; "
                                   "mxfp4 B=4 and fp8 B=32, 64 index heads x 128", "iters": iters},
            "cases": out}


# ---- the module path (and a module decode step at config-2 dimensions) ----

MODULE_C1 = dict(hidden_size=512, num_attention_heads=8, head_dim=160, qk_rope_head_dim=32, q_lora_rank=256,
                 o_groups=2, o_lora_rank=128, index_n_heads=4, index_head_dim=64, index_topk=128, compress_ratio=4,
                 sliding_window=64, seq=1024, batch=1, seed=0)
# config-2 dimensions for the attention; hidden / low-rank sizes are not named by the config
MODULE_C2 = dict(hidden_size=4096, num_attention_heads=128, head_dim=576, qk_rope_head_dim=64, q_lora_rank=1536,
                 o_groups=16, o_lora_rank=1024, index_n_heads=64, index_head_dim=128, index_topk=2048,
                 compress_ratio=4, sliding_window=128, ctx=32768, batch=32, seed=6)


def module_param_shapes(c):
    """name -> shape of the parameters of DeepseekV41Attention for a KV + index source
    layer (owlet1/attention.py:106-127, cache.py:134-140, indexer.py:63-76)."""
    h, d, hid, ql = c["num_attention_heads"], c["head_dim"], c["hidden_size"], c["q_lora_rank"]
    hi, di, og, orank = c["index_n_heads"], c["index_head_dim"], c["o_groups"], c["o_lora_rank"]
    return {"wq_a.weight": (ql, hid), "q_norm.weight": (ql,), "wq_b.weight": (h * d, ql), "wkv.weight": (d, hid),
            "kv_norm.weight": (d,), "wo_a.weight": (og * orank, h * d // og), "wo_b.weight": (hid, og * orank),
            "attn_sink": (h,), "compressor.wkv.weight": (d, hid), "compressor.wgate.weight": (d, hid),
            "compressor.norm.weight": (d,), "indexer.wq_b.weight": (hi * di, ql),
            "indexer.weights_proj.weight": (hi, hid), "indexer.wk.weight": (di, d), "indexer.k_norm.weight": (di,)}


def module_layer(torch, dev, c, dtype):
    """(DeepseekV41Attention on `dev` in `dtype`, its fp32 parameters on the CPU): every
    weight and the sink ~N(0, 0.02), norm weights 1 (BASELINE config 1's initialisation)."""
    from mzoo_amd import owlet1 as MO
    cfg = MO.AttentionConfig(
        hidden_size=c["hidden_size"], num_attention_heads=c["num_attention_heads"], head_dim=c["head_dim"],
        qk_rope_head_dim=c["qk_rope_head_dim"], q_lora_rank=c["q_lora_rank"], o_groups=c["o_groups"],
        o_lora_rank=c["o_lora_rank"], rope_theta=ROPE_THETA, compress_rope_theta=COMPRESS_ROPE_THETA,
        sliding_window=c["sliding_window"], compress_ratios=[c["compress_ratio"]], kv_source_layer_ids=[0],
        index_source_layer_ids=[0], candidate_source_layer_id=-1, index_n_heads=c["index_n_heads"],
        index_head_dim=c["index_head_dim"], index_topk=c["index_topk"], rms_norm_eps=1e-20)
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    params = {}
    for name, shape in sorted(module_param_shapes(c).items()):
        params[name] = (torch.ones(shape, device=dev) if name.endswith("norm.weight")
                        else torch.randn(shape, generator=gen, device=dev) * 0.02)
    mod = MO.DeepseekV41Attention(cfg, 0)
    mod.load_state_dict({k: v.cpu() for k, v in params.items()}, strict=True)
    return mod.to(device=dev, dtype=dtype).eval(), params, gen


def module_decode_step(torch, dev, steps, warmup):
    """One module decode step at config-2 dimensions: DeepseekV41Attention.forward on one
    new token per row of B=32 through DeepseekV41CSACache holding a context of 32767 tokens
    (8191 compressed groups + the carried partial group, the last 127 window entries, the
    MXFP4-packed keys), bf16 model, no mask; the steps advance to position 32767."""
    from transformers.cache_utils import Cache

    from mzoo_amd import owlet1 as MO
    from mzoo_amd import quant
    c = MODULE_C2
    mod, _, gen = module_layer(torch, dev, c, torch.bfloat16)
    cfg = mod.config
    b, d, di, r, w = c["batch"], c["head_dim"], c["index_head_dim"], c["compress_ratio"], c["sliding_window"]
    start = c["ctx"] - 1 - warmup - steps
    cache = Cache(layers=[MO.DeepseekV41CSACache(cfg)])
    layer = cache.layers[0]
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev)  # noqa: E731
    win = rnd(b, 1, w - 1, d).bfloat16()
    layer.update(win, win)
    layer.cumulative_length = start
    g0 = start // r
    layer._store["compressor"].append(rnd(b, g0, d).bfloat16())   # a bf16 model's cache is read in place
    keys = rnd(b, g0, di).bfloat16()
    layer._store["indexer"].append(keys)
    layer.append_packed_index_k(*quant.quant_mxfp4(keys))
    layer.entry_count["compressor"] = g0
    layer.buffer_kv["compressor"] = rnd(b, start - g0 * r, d)
    layer.buffer_gate["compressor"] = rnd(b, start - g0 * r, d)
    rot = MO.DeepseekV41RotaryEmbedding(cfg).to(dev)
    xs = [rnd(b, 1, c["hidden_size"]).bfloat16() for _ in range(4)]

    def one(i):
        pos = torch.full((b, 1), start + i, dtype=torch.int64, device=dev)
        x = xs[i % len(xs)]
        pe = {"main": rot(x, pos, "main"), "compress": rot(x, pos, "compress")}
        with torch.no_grad():
            return mod(x, position_embeddings=pe, attention_mask=None, past_key_values=cache,
                       shared=MO.SharedState(), position_ids=pos)[0]

    for i in range(warmup):
        one(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup, warmup + steps):
        one(i)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    weight_bytes = sum(p.numel() * p.element_size() for p in mod.parameters())
    return {"ms_per_step": ms, "tokens_per_s": b / (ms * 1e-3), "batch": b, "context": c["ctx"],
            "steps": steps, "weight_bytes": weight_bytes,
            "workload": "DeepseekV41Attention.forward, one token per row, B=32 at context 32768 (positions "
                        f"{start + warmup}..{start + warmup + steps - 1}), 128 heads x (512+64), indexer 64x128 "
                        "MXFP4 over 8191-8192 groups, top-2048, window 128, bf16 weights (hidden 4096, q rank 1536, "
                        "16 output groups of rank 1024), eager launches, no mask",
            "note": "includes the projections (the weights are read once per step) and the host's launch "
                    "overhead of the eager module; the graph-captured kernel step is the --config 2 line"}


def run_module(torch, dev, args):
    """the module drop-in's layer forward (no cache) over B=1, S=1024."""
    from mzoo_amd import owlet1 as MO
    c = MODULE_C1
    mod, params, gen = module_layer(torch, dev, c, torch.float32)
    b, s = c["batch"], c["seq"]
    x = torch.randn(b, s, c["hidden_size"], generator=gen, device=dev)
    pos = torch.arange(s, device=dev).unsqueeze(0).expand(b, -1).contiguous()
    rot = MO.DeepseekV41RotaryEmbedding(mod.config).to(dev)
    w = c["sliding_window"]
    kk = torch.arange(s, device=dev)
    band = (kk[None, :] <= kk[:, None]) & (kk[None, :] > kk[:, None] - w)
    mask = torch.zeros(b, 1, s, s, device=dev).masked_fill_(~band, torch.finfo(torch.float32).min)

    def fwd(m=None):
        pe = {"main": rot(x, pos, "main"), "compress": rot(x, pos, "compress")}
        with torch.no_grad():
            return mod(x, position_embeddings=pe, attention_mask=m, past_key_values=None, shared=MO.SharedState(),
                       position_ids=pos)[0]

    def timed(m, n):
        for _ in range(3):
            fwd(m)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fwd(m)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e3

    steps = max(5, min(args.steps, 50))
    ms = timed(None, steps)
    ms_mask = timed(mask, steps)

    # the attention kernel alone (its inputs at the layer's shapes), back-to-back launches
    from mzoo_amd import indexer as IDX
    h, d, k, r = c["num_attention_heads"], c["head_dim"], c["index_topk"], c["compress_ratio"]
    g = s // r
    q = torch.randn(b, s, h, d, generator=gen, device=dev).bfloat16()
    full = torch.randn(b, s, d, generator=gen, device=dev).bfloat16()
    comp = torch.randn(b, g, d, generator=gen, device=dev).bfloat16()
    sc = torch.randn(b, s, g, generator=gen, device=dev)
    sc = sc.masked_fill(torch.arange(g, device=dev)[None, None, :] >= (pos[..., None] + 1) // r, float("-inf"))
    idx = IDX.topk(sc, k)
    sinks = torch.randn(h, generator=gen, device=dev)
    rel = pos.reshape(-1)
    t_attn = graph_time(torch, [lambda: MO._sparse_attend(q, sinks, window=(full, rel, w), parts=[(comp, idx)])],
                        64)
    t = torch.arange(s, dtype=torch.float64)
    pairs = float((torch.clamp(t + 1, max=w) + torch.clamp((t + 1) // r, max=k)).sum())
    attn_flops = 4.0 * d * h * pairs
    attn_bytes = 2.0 * s * h * d * 2 + (s + g) * d * 2 + s * k * 4
    roof = roofline(None, attn_flops, attn_bytes, t_attn)
    roof.update({"traffic": None, "kernel": "sparse_mqa (D=160, 8 heads)", "kernel_us": t_attn})

    cpu = None
    if not args.no_cpu:
        from oracle import model as OM
        torch.set_num_threads(os.cpu_count() or 1)
        cp = {k_: v.float().cpu() for k_, v in params.items()}
        ocfg = dict(c, rms_norm_eps=1e-20, compress_rope_theta=COMPRESS_ROPE_THETA)
        xc, pc = x.cpu(), pos.cpu()
        times = []
        t_start = time.perf_counter()
        while len(times) < 5 and (time.perf_counter() - t_start < args.cpu_seconds or len(times) < 2):
            t0 = time.perf_counter()
            OM.layer_forward(cp, ocfg, xc, pc)
            times.append(time.perf_counter() - t0)
        times.sort()
        med = times[len(times) // 2]
        cpu = {"value": s / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"the whole config-1 layer forward (B=1, S=1024; the oracle's module composition in fp32), "
                         f"median of {len(times)} runs"}
    dec = module_decode_step(torch, dev, steps=max(5, min(args.steps, 20)), warmup=3)
    return {
        "metric": METRIC,
        "value": s * b / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 3,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 weights and projections; bf16 attention (MFMA), FP8 / FP4 fake-quantized caches",
        "data": "synthetic (seed 0): weights ~N(0, 0.02), norm weights 1, hidden states ~N(0, 1), on the GPU",
        "config": {"workload": "config1: DeepseekV41Attention.forward (mzoo_amd drop-in) over B=1 S=1024, 8 heads x "
                               "(128+32) latent, indexer 4x64 MXFP4, ratio 4, top-128, window 64, sink, no cache, "
                               "eager launches",
                   "batch": b, "seq_len": s, "heads": h, "topk": k, "window": w,
                   "step": "one layer forward without a mask (the window in token order); "
                           "ms_with_mask: with the model's sliding causal mask"},
        "ms_with_mask": ms_mask,
        "roofline": roof,
        "cpu_baseline": cpu,
        "module_decode_c2": dec,
    }


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs are not part of it "
              f"(got --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    from mzoo_amd import csa2_attn
    csa2_attn.set_merge(1 if args.merge == "inline" else 0)
    if args.copy_mib:
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4}))
        return
    if args.kernels:
        print(json.dumps(run_kernels(torch, dev, args)))
        return
    if args.reindex:
        print(json.dumps(run_reindex(torch, dev, args)))
        return
    if args.config == 1:
        out = run_module(torch, dev, args)
    elif args.config == 3:
        out = run_prefill(torch, dev, args)
    else:
        out = run_decode(torch, dev, args)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
