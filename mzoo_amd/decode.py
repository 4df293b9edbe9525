"""Graph-captured decode step of one CSA2 attention layer (piece 6).

Replaces the per-step work of ``DeepseekV41Attention.forward`` with a cache
(``owlet1/attention.py:145-229``; cache state ``owlet1/cache.py:84-124``; indexer
``owlet1/indexer.py:78-165``) for one new token per batch row, with every piece of state
preallocated on the device so the whole step records into one HIP graph:

* window ring  ``win``   uint8 [B, W, 656]  -- FP8-b128 latent of the last W tokens,
  token t at slot t % W (the reference keeps the last W-1 and concatenates the new one,
  ``cache.py:84-94``; the ring holds the same W entries without a ``torch.cat``);
* compressed   ``main``  uint8 [B, Gcap, 656] -- one entry per emitted group;
* indexer keys ``k_*``   FP8 (codes [B,Gcap,Di] + fp32 scale [B,Gcap]) or MXFP4
  (nibbles [B,Gcap,Di/2] + e8m0 [B,Gcap,Di/32]);
* optional dense coarse branch ``coarse`` uint8 [B, Gc, 656] (hierarchical config);
* ``positions`` int64 [B] on the device: the position of the token being decoded.  The
  reference keeps Python ints (``entry_count``, ``cache.py:46``) and grows tensors with
  ``torch.cat``; here visibility is derived on the device from ``positions``
  (``(pos+1) // ratio`` visible groups, ``indexer.py:141-143``), so nothing on the host
  changes between steps.

``step(q, kv, q_idx, w)`` for one token per row:
  1-3. FP8 index: one launch packs the new token's latent into its ring slot (derived on
     the device from ``positions``), quantizes the indexer query (FP8 b128 per head) and
     scores all keys (group-causal ``-inf`` beyond ``(pos+1)//ratio``); MXFP4 index: the
     append + quantization launch, then the scores launch,
  4. top-k (lowest index wins ties),
  5. sparse MQA over window + [coarse] + top-k entries with the sink, split-KV + merge,
  6. ``positions += 1`` when ``advance`` (by the merge launch of step 5, no launch of its own).

Group emission -- the compressor, the cache append and the indexer's key publication, one
entry per ``ratio`` tokens (``owlet1/cache.py:96-124``, ``:159-172``, ``owlet1/indexer.py:96-117``,
``owlet1/attention.py:173-192``) -- runs inside the step when the layer has its
``CompressorWeights`` and the step gets the token's fp32 compressor projections
(``step(..., compress=(kv, gate))``): a first launch writes them to a device carry ring and,
when the token completes a group, pools the group, normalizes it, writes its rotated FP8-b128
entry and its index key, before the indexer scores the keys -- so a graph replay that
advances the positions emits groups itself.  The same launch copies the token's RoPE tables
out of a position-indexed device table (``rope="table"``), so nothing on the host changes
between replays.  ``append_groups`` writes groups from the host (prefill).

With ``rope=(cos, sin, index_cos, index_sin)`` (bf16 [B, 32] each: the new token's
``position_embeddings`` and the indexer's compress-RoPE tables) the step also takes over the
per-token prologue and epilogue of ``DeepseekV41Attention.forward``: q and q_idx arrive
unrotated, kv is the raw ``wkv`` projection (RMSNorm with ``kv_norm_weight``, RoPE and the
window append happen in the indexer launch, ``attention.py:147-155``, ``indexer.py:126-128``),
q is rotated as the attention kernel loads it, and the output carries the inverse rotation
(``attention.py:226``) -- the same four launches as without it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib, csa2_attn, indexer, quant
from .rope import rope_inv_freq


class GroupedOutputProjection:
    """The attention output's projection, ``wo_b(wo_a(o.reshape(..., G, -1)).flatten(-2))``:
    ``DeepseekV41GroupedLinear`` (owlet1/attention.py:20-39; a block-diagonal projection of
    each of the ``o_groups`` head groups to ``o_lora_rank``) then ``wo_b``
    (owlet1/attention.py:233-235).  Both are plain GEMMs and run on hipBLASLt (torch's
    ``bmm`` / ``linear``); the grouped weight is stored once as ``[G, H*D/G, r]``, so the
    batched product's right operand is contiguous.  Input: o [..., H, D] with the inverse
    RoPE already applied (what ``SparseDecodeLayer.step(..., rope=...)`` returns)."""

    def __init__(self, wo_a_weight: torch.Tensor, wo_b_weight: torch.Tensor, o_groups: int):
        g = o_groups
        if wo_a_weight.shape[0] % g or wo_b_weight.shape[1] != wo_a_weight.shape[0]:
            raise ValueError("GroupedOutputProjection: wo_a [G*r, H*D/G] and wo_b [hidden, G*r] expected")
        self.groups = g
        self.rank = wo_a_weight.shape[0] // g
        self.in_per_group = wo_a_weight.shape[1]
        self.wa = wo_a_weight.view(g, self.rank, self.in_per_group).transpose(1, 2).contiguous()
        self.wb = wo_b_weight.contiguous()

    def __call__(self, o: torch.Tensor) -> torch.Tensor:
        lead = o.shape[:-2]
        x = o.reshape(-1, self.groups, self.in_per_group).transpose(0, 1).contiguous()  # [G, N, H*D/G]
        y = torch.bmm(x, self.wa)                                                         # [G, N, r]
        y = y.transpose(0, 1).reshape(*lead, self.groups * self.rank)
        return torch.nn.functional.linear(y, self.wb)


@dataclass
class CompressorWeights:
    """What the in-step group emission reads: the compressor's RMSNorm weight
    (``owlet1/cache.py:140``), the indexer's key projection ``wk`` [Di, D] and ``k_norm`` weight
    (``owlet1/indexer.py:75-76``), their epsilons, the coarse branch's compressor norm weight
    (hierarchical config), and the compress RoPE the group positions rotate with: its base
    (``compress_rope_theta``, ``owlet1/config.py:238``) and, when the model extends its context
    with YaRN (``owlet1/config.py:419-434``), the YaRN settings (the keywords of
    ``mzoo_amd.rope.yarn_inv_freq``)."""
    norm_weight: torch.Tensor
    wk: torch.Tensor
    k_norm_weight: torch.Tensor
    eps: float = 1e-6
    k_eps: float = 1e-6
    coarse_norm_weight: torch.Tensor | None = None
    rope_theta: float = 160000.0
    rope_yarn: dict | None = None


def rope_table(positions: int, rope_dim: int, theta: float, yarn: dict | None = None) -> torch.Tensor:
    """bf16 [positions, rope_dim]: row p holds the cos (first rope_dim/2) and sin of position
    p, as ``DeepseekV41RotaryEmbedding.forward`` computes them (``owlet1/norm_rope.py:108-124``:
    ``inv_freq`` of the default RoPE or of YaRN, ``pos * inv_freq`` in fp32, cos / sin times
    the attention factor, then the activations' dtype), on the CPU."""
    inv, scale = rope_inv_freq(theta, rope_dim, yarn)
    freqs = torch.arange(positions, dtype=torch.float).view(-1, 1) * inv.view(1, -1)
    return torch.cat([freqs.cos() * scale, freqs.sin() * scale], -1).to(torch.bfloat16)


@dataclass
class DecodeConfig:
    batch: int
    heads: int = 128
    nope: int = 512
    rope: int = 64
    index_heads: int = 64
    index_dim: int = 128
    ratio: int = 4
    window: int = 128
    topk: int = 2048
    max_groups: int = 8192
    index_format: str = "fp8"       # "fp8" or "mxfp4"
    coarse_ratio: int = 0            # > 0: dense coarse branch (hierarchical config)
    coarse_groups: int = 0
    nsplit: int = 4
    # run the window and dense branches of the attention on a second stream, beside the
    # top-k (which they do not depend on); the top-k entries follow on the main one.  Off by
    # default: replayed in a graph the extra launch and the join cost more than the overlap
    # gains (config 2: 86.5 vs 74.3 us per layer, config 5: 83.9 vs 77.5)
    branch_overlap: bool = False
    # with in-step emission (rope="table") and ratio 4: the emission (both branches) joins the
    # indexer launch (one workgroup per row emits the group and scores the new key, nine pool
    # a coarse group) -- one launch less per step; False keeps the emission launch of its own
    merged_emit: bool = True
    # the top-k inside the attention launch (every attention workgroup of a row selects the
    # row's list from the scores itself: no top-k launch) where the attention kernel takes it
    # -- at most 8192 keys and a top-2048, multiples of 4; False keeps the top-k launch
    select_in_attention: bool = True

    @property
    def dim(self) -> int:
        return self.nope + self.rope


class SparseDecodeLayer:
    def __init__(self, cfg: DecodeConfig, device, sinks: torch.Tensor | None = None,
                 kv_norm_weight: torch.Tensor | None = None, kv_norm_eps: float = 1e-6,
                 out_proj: GroupedOutputProjection | None = None, compressor: CompressorWeights | None = None,
                 max_position: int | None = None):
        if cfg.index_format not in ("fp8", "mxfp4"):
            raise ValueError(f"index_format must be 'fp8' or 'mxfp4', got {cfg.index_format!r}")
        if cfg.index_format == "fp8" and cfg.index_dim != 128:
            raise ValueError(f"the FP8 index (one b128 block per head) needs index_dim 128, got {cfg.index_dim}")
        self.cfg = cfg
        self.device = torch.device(device)
        b, eb = cfg.batch, quant.entry_bytes(cfg.nope, cfg.rope)
        u8 = dict(dtype=torch.uint8, device=self.device)
        self.win = torch.zeros(b, cfg.window, eb, **u8)
        self.main = torch.zeros(b, cfg.max_groups, eb, **u8)
        self.coarse = torch.zeros(b, cfg.coarse_groups, eb, **u8) if cfg.coarse_ratio else None
        di = cfg.index_dim
        if cfg.index_format == "fp8":
            self.k_codes = torch.zeros(b, cfg.max_groups, di, **u8)
            self.k_scales = torch.ones(b, cfg.max_groups, dtype=torch.float32, device=self.device)
        else:
            self.k_packed = torch.zeros(b, cfg.max_groups, di // 2, **u8)
            self.k_e8m0 = torch.full((b, cfg.max_groups, di // 32), 127, **u8)
        self.positions = torch.zeros(b, dtype=torch.int64, device=self.device)
        self.sinks = None if sinks is None else sinks.float().to(self.device).contiguous()
        self.kv_norm_weight = None if kv_norm_weight is None else \
            kv_norm_weight.to(device=self.device, dtype=torch.bfloat16).contiguous()
        self.kv_norm_eps = float(kv_norm_eps)
        self.out_proj = out_proj  # with it, step(..., rope=...) returns the projected output
        # per-step buffers (fixed addresses, so a captured graph can replay them)
        self.scores = torch.empty(b, 1, cfg.max_groups, dtype=torch.float32, device=self.device)
        self.idx = torch.empty(b, cfg.topk, dtype=torch.int32, device=self.device)
        self.topk_ws = torch.empty(max(indexer.topk_workspace_bytes(b, cfg.max_groups), 16), dtype=torch.uint8,
                                   device=self.device)
        self.out = torch.empty(b, cfg.heads, cfg.dim, dtype=torch.bfloat16, device=self.device)
        self.lse = torch.empty(b, cfg.heads, dtype=torch.float32, device=self.device)
        # splits of the window + dense branches (about 256 entries each) and of the top-k entries
        self.nsplit_wd = max(1, -(-(cfg.window + cfg.coarse_groups) // 256)) if cfg.branch_overlap else 0
        self.workspace = csa2_attn.new_workspace(b, cfg.heads, cfg.dim, cfg.nsplit + self.nsplit_wd, self.device)
        self._side = torch.cuda.Stream(device=self.device) if cfg.branch_overlap else None
        self._slot_base = torch.arange(b, device=self.device, dtype=torch.int64) * cfg.window
        hi = cfg.index_heads
        if cfg.index_format == "mxfp4":  # the FP8 step quantizes the query inside its indexer launch
            self.q_codes = torch.empty(b, 1, hi, di // 2, **u8)
            self.q_e8m0 = torch.empty(b, 1, hi, di // 32, **u8)
        self._graph = None
        self._static = None
        self._graph_advances = False
        self.rope_table = None
        self._pos_max = None  # host copy of the largest row position (None: not set from the host)
        self.compressor = None
        if compressor is not None:
            self._init_emission(compressor, max_position)

    def _init_emission(self, cw: CompressorWeights, max_position: int | None) -> None:
        cfg = self.cfg
        b, d, dev = cfg.batch, cfg.dim, self.device
        if cfg.index_dim != 128 or cfg.nope != 512 or cfg.rope != 64:
            raise ValueError("in-step emission: latent 512 + 64 and index keys of 128 channels")
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.compressor = CompressorWeights(
            norm_weight=cw.norm_weight.to(**bf).contiguous(), wk=cw.wk.to(**bf).contiguous(),
            k_norm_weight=cw.k_norm_weight.to(**bf).contiguous(), eps=float(cw.eps), k_eps=float(cw.k_eps),
            coarse_norm_weight=None if cw.coarse_norm_weight is None else cw.coarse_norm_weight.to(**bf).contiguous(),
            rope_theta=float(cw.rope_theta), rope_yarn=None if cw.rope_yarn is None else dict(cw.rope_yarn))
        if tuple(self.compressor.wk.shape) != (cfg.index_dim, d):
            raise ValueError(f"in-step emission: wk must be [{cfg.index_dim}, {d}]")
        if cfg.coarse_ratio and self.compressor.coarse_norm_weight is None:
            raise ValueError("in-step emission: the coarse branch needs coarse_norm_weight")
        f32 = dict(dtype=torch.float32, device=dev)
        self.carry_kv = torch.zeros(b, cfg.ratio, d, **f32)
        self.carry_gate = torch.zeros(b, cfg.ratio, d, **f32)
        if cfg.coarse_ratio:
            self.coarse_carry_kv = torch.zeros(b, cfg.coarse_ratio, d, **f32)
            self.coarse_carry_gate = torch.zeros(b, cfg.coarse_ratio, d, **f32)
        npos = max_position or max(cfg.max_groups * cfg.ratio, cfg.coarse_groups * max(cfg.coarse_ratio, 1)) + 1
        self.rope_table = rope_table(npos, cfg.rope, self.compressor.rope_theta,
                                     self.compressor.rope_yarn).to(dev).contiguous()
        self.step_cos = torch.zeros(b, cfg.rope // 2, **bf)
        self.step_sin = torch.zeros(b, cfg.rope // 2, **bf)
        # 64 indexer heads: the emission launch also runs the step's prologue (window entry,
        # the indexer query's RoPE and quantization) and the indexer is the plain scorer
        self._emit_prologue = cfg.index_heads == 64
        # the emission inside the indexer launch (coarse branches of ratio <= 128, up to 1024 rows)
        self._merged_emit = (self._emit_prologue and cfg.merged_emit and cfg.ratio == 4
                             and (not cfg.coarse_ratio or (2 <= cfg.coarse_ratio <= 128 and b <= 1024)))
        # the merged launch's key-projection handoff between a row's two lead workgroups
        # (zero before the first step; the launch keeps its per-row count there)
        self.key_half = torch.zeros(b, 40, dtype=torch.int64, device=dev) if self._merged_emit else None
        if self._emit_prologue and cfg.index_format == "fp8":
            self.q_codes = torch.empty(b, 1, cfg.index_heads, cfg.index_dim, dtype=torch.uint8, device=dev)
            self.q_scales = torch.empty(b, 1, cfg.index_heads, dtype=torch.float32, device=dev)

    # ---- state ---------------------------------------------------------------------------
    def set_positions(self, pos) -> None:
        p = torch.as_tensor(pos, dtype=torch.int64)
        self._pos_max = int(p.max())
        self._check_table()
        self.positions.copy_(p.to(self.device).expand(self.cfg.batch))

    def _check_table(self) -> None:
        """The emission reads the token's RoPE tables from row `pos` of the position table
        and skips rows beyond it (their window entry and quantized query would keep the
        previous step's contents): refuse a step at a position the table does not hold."""
        if self.rope_table is not None and self._pos_max is not None and self._pos_max >= self.rope_table.shape[0]:
            raise ValueError(f"SparseDecodeLayer: position {self._pos_max} is beyond the RoPE position table "
                             f"({self.rope_table.shape[0]} rows; raise max_position)")

    def fill_window(self, latents: torch.Tensor, last_position: int) -> None:
        """latents [B, W, D] for tokens last_position-W+1 .. last_position."""
        w = self.cfg.window
        toks = torch.arange(last_position - w + 1, last_position + 1, device=self.device)
        slots = (self._slot_base.view(-1, 1) + (toks % w).view(1, -1)).reshape(-1)
        quant.pack_latent_fp8_b128(latents.reshape(-1, self.cfg.dim), rope=self.cfg.rope,
                                   out=self.win.view(-1, self.win.shape[-1]), dst_index=slots)

    def append_groups(self, start: int, latents: torch.Tensor, index_keys: torch.Tensor) -> None:
        """Write groups start..start+n-1: rotated latents [B,n,D] into the main cache and
        their indexer keys [B,n,Di] (quantized here) -- update_compressor_states."""
        n = latents.shape[1]
        rows = (torch.arange(self.cfg.batch, device=self.device).view(-1, 1) * self.cfg.max_groups
                + torch.arange(start, start + n, device=self.device).view(1, -1)).reshape(-1)
        quant.pack_latent_fp8_b128(latents.reshape(-1, self.cfg.dim), rope=self.cfg.rope,
                                   out=self.main.view(-1, self.main.shape[-1]), dst_index=rows)
        if self.cfg.index_format == "fp8":
            codes, scales = quant.quant_fp8_block(index_keys, self.cfg.index_dim)
            self.k_codes[:, start:start + n] = codes
            self.k_scales[:, start:start + n] = scales[..., 0]
        else:
            packed, e8 = quant.quant_mxfp4(index_keys)
            self.k_packed[:, start:start + n] = packed
            self.k_e8m0[:, start:start + n] = e8

    def set_carry(self, kv: torch.Tensor, gate: torch.Tensor, coarse: bool = False) -> None:
        """The partial group carried into the next step (prefill): kv / gate fp32 [B, n, D],
        the compressor projections of the last n tokens before the current position, n =
        position % ratio -- store_compression_weights' buffer (owlet1/cache.py:96-113)."""
        ratio = self.cfg.coarse_ratio if coarse else self.cfg.ratio
        ck, cg = (self.coarse_carry_kv, self.coarse_carry_gate) if coarse else (self.carry_kv, self.carry_gate)
        n = kv.shape[1]
        if n >= ratio:
            raise ValueError(f"set_carry: a partial group holds fewer than {ratio} tokens, got {n}")
        ck[:, :n] = kv.float()
        cg[:, :n] = gate.float()

    def _emit(self, compress, rope_from_table: bool, prologue=None) -> None:
        """The in-step emission launch (both compressed branches in one when there is a coarse
        branch: ``mzk_decode_emit_pair``), see the module doc.
        ``prologue`` = (kv projection bf16 [B, D], indexer query bf16 [B, 64, Di]): the first
        launch also writes the token's window entry and the quantized indexer query."""
        cfg, cw = self.cfg, self.compressor
        b = cfg.batch
        st = _lib.stream_of(self.positions)
        fp8 = cfg.index_format == "fp8"
        kv, gate = (t.contiguous() for t in compress[:2])
        for t in (kv, gate):
            if t.dtype != torch.float32 or t.shape != (b, cfg.dim):
                raise ValueError(f"step(compress=...): fp32 [{b}, {cfg.dim}] projections expected")
        keys = (self.k_codes, self.k_scales) if fp8 else (self.k_packed, self.k_e8m0)
        tabs = (self.step_cos.data_ptr(), self.step_sin.data_ptr()) if rope_from_table else (None, None)
        pro = (None, None, 0.0, None, 0, 0, None, 0, None, None)
        if prologue is not None:
            pkv, pq = prologue
            if pkv.dtype != torch.bfloat16 or pkv.shape != (b, cfg.dim) or not pkv.is_contiguous():
                raise ValueError(f"step: kv must be a contiguous bf16 [{b}, {cfg.dim}] projection")
            if pq.dtype != torch.bfloat16 or pq.shape != (b, cfg.index_heads, cfg.index_dim) \
                    or not pq.is_contiguous():
                raise ValueError(f"step: q_idx must be a contiguous bf16 [{b}, {cfg.index_heads}, "
                                 f"{cfg.index_dim}] tensor")
            _lib.require_gpu(pkv, pq)
            qs = self.q_scales if fp8 else self.q_e8m0
            pro = (pkv.data_ptr(), self.kv_norm_weight.data_ptr(), self.kv_norm_eps, self.win.data_ptr(),
                   cfg.window, cfg.window, pq.data_ptr(), 0 if fp8 else 1, self.q_codes.data_ptr(), qs.data_ptr())
        fine = (self.positions.data_ptr(), b, kv.data_ptr(), gate.data_ptr(),
                self.carry_kv.data_ptr(), self.carry_gate.data_ptr(), cfg.ratio, cw.norm_weight.data_ptr(), cw.eps,
                self.main.data_ptr(), cfg.max_groups, cfg.max_groups, cw.wk.data_ptr(),
                cw.k_norm_weight.data_ptr(), cw.k_eps, 0 if fp8 else 1, keys[0].data_ptr(), keys[1].data_ptr(),
                cfg.max_groups, self.rope_table.data_ptr(), self.rope_table.shape[0], *tabs, *pro)
        if not cfg.coarse_ratio:
            _lib.call("mzk_decode_emit", *fine, st)
            return
        if len(compress) != 4:
            raise ValueError("step(compress=...): the coarse branch needs (kv, gate, coarse_kv, coarse_gate)")
        ckv, cg = (t.contiguous() for t in compress[2:])
        for t in (ckv, cg):
            if t.dtype != torch.float32 or t.shape != (b, cfg.dim):
                raise ValueError(f"step(compress=...): fp32 [{b}, {cfg.dim}] projections expected")
        # both compressors in one launch (the coarse branch has no key, prologue or step tables)
        _lib.call("mzk_decode_emit_pair", *fine, ckv.data_ptr(), cg.data_ptr(), self.coarse_carry_kv.data_ptr(),
                  self.coarse_carry_gate.data_ptr(), cfg.coarse_ratio, cw.coarse_norm_weight.data_ptr(), cw.eps,
                  self.coarse.data_ptr(), cfg.coarse_groups, cfg.coarse_groups, st)

    def _emit_scores(self, compress, kv, q_idx, w) -> None:
        """The emission and the indexer scores in one launch (``mzk_decode_emit_scores``): per
        row one workgroup carries the token and emits a completed group (scoring its new key
        itself), one writes the window entry, and the scoring workgroups rotate and quantize
        the indexer query themselves."""
        cfg, cw = self.cfg, self.compressor
        b = cfg.batch
        fp8 = cfg.index_format == "fp8"
        if len(compress) != (4 if cfg.coarse_ratio else 2):
            raise ValueError("step(compress=...): (kv, gate[, coarse_kv, coarse_gate]) for the layer's branches")
        ckv, gate = (t.contiguous() for t in compress[:2])
        coarse = (None,) * 4 + (0, None, 0.0, None, 0, 0)
        if cfg.coarse_ratio:
            c_kv, c_gate = (t.contiguous() for t in compress[2:])
            for t in (c_kv, c_gate):
                if t.dtype != torch.float32 or t.shape != (b, cfg.dim):
                    raise ValueError(f"step(compress=...): fp32 [{b}, {cfg.dim}] projections expected")
            _lib.require_gpu(c_kv, c_gate)
            coarse = (c_kv.data_ptr(), c_gate.data_ptr(), self.coarse_carry_kv.data_ptr(),
                      self.coarse_carry_gate.data_ptr(), cfg.coarse_ratio, cw.coarse_norm_weight.data_ptr(), cw.eps,
                      self.coarse.data_ptr(), cfg.coarse_groups, cfg.coarse_groups)
        for t in (ckv, gate):
            if t.dtype != torch.float32 or t.shape != (b, cfg.dim):
                raise ValueError(f"step(compress=...): fp32 [{b}, {cfg.dim}] projections expected")
        if kv.dtype != torch.bfloat16 or kv.shape != (b, cfg.dim):
            raise ValueError(f"step: kv must be a contiguous bf16 [{b}, {cfg.dim}] projection")
        if q_idx.dtype != torch.bfloat16 or q_idx.shape != (b, cfg.index_heads, cfg.index_dim):
            raise ValueError(f"step: q_idx must be a contiguous bf16 [{b}, {cfg.index_heads}, {cfg.index_dim}] tensor")
        wc = w.reshape(b, cfg.index_heads)
        if wc.dtype != torch.float32:
            raise ValueError("step: w must be fp32")
        wc = wc.contiguous()
        _lib.require_gpu(ckv, gate, kv, q_idx, wc)
        keys = (self.k_codes, self.k_scales) if fp8 else (self.k_packed, self.k_e8m0)
        _lib.call("mzk_decode_emit_scores", self.positions.data_ptr(), b, ckv.data_ptr(), gate.data_ptr(),
                  self.carry_kv.data_ptr(), self.carry_gate.data_ptr(), cfg.ratio, cw.norm_weight.data_ptr(), cw.eps,
                  self.main.data_ptr(), cfg.max_groups, cfg.max_groups, cw.wk.data_ptr(), cw.k_norm_weight.data_ptr(),
                  cw.k_eps, 0 if fp8 else 1, keys[0].data_ptr(), keys[1].data_ptr(), cfg.max_groups,
                  self.rope_table.data_ptr(), self.rope_table.shape[0], self.step_cos.data_ptr(),
                  self.step_sin.data_ptr(), kv.data_ptr(), self.kv_norm_weight.data_ptr(), self.kv_norm_eps,
                  self.win.data_ptr(), cfg.window, cfg.window, q_idx.data_ptr(), wc.data_ptr(), cfg.index_heads,
                  cfg.max_groups, self.scores.data_ptr(), cfg.max_groups, *coarse, self.key_half.data_ptr(),
                  _lib.stream_of(self.positions))

    def fill_coarse(self, latents: torch.Tensor) -> None:
        """latents [B, n, D] -> coarse entries 0..n-1 of every row."""
        n = latents.shape[1]
        rows = (torch.arange(self.cfg.batch, device=self.device).view(-1, 1) * self.cfg.coarse_groups
                + torch.arange(n, device=self.device).view(1, -1)).reshape(-1)
        quant.pack_latent_fp8_b128(latents.reshape(-1, self.cfg.dim), rope=self.cfg.rope,
                                   out=self.coarse.view(-1, self.coarse.shape[-1]), dst_index=rows)

    # ---- the step ------------------------------------------------------------------------
    def step(self, q: torch.Tensor, kv: torch.Tensor | None, q_idx: torch.Tensor, w: torch.Tensor,
             advance: bool = False, rope: tuple | str | None = None, compress: tuple | None = None) -> torch.Tensor:
        """q bf16 [B,H,D] (rotated), kv bf16 [B,D] (the new token's rotated latent, or None
        if already in the ring), q_idx bf16 [B,Hi,Di] (rotated), w fp32 [B,Hi] (x Hi^-0.5).
        With ``rope`` (see the module docstring) q, q_idx are unrotated, kv is the raw
        projection, and the returned output has the inverse rotation applied; ``rope="table"``
        takes the four tables from the device table at the rows' positions (needs the
        layer's ``CompressorWeights``).  ``compress`` = (kv, gate[, coarse_kv, coarse_gate]):
        the token's fp32 compressor projections [B, D], emitted into the caches in the step."""
        if compress is not None or rope == "table":
            self._check_table()
        out = self._step(q, kv, q_idx, w, advance, rope, compress)
        if advance and self._pos_max is not None:
            self._pos_max += 1
        return out

    def _step(self, q, kv, q_idx, w, advance, rope, compress):
        cfg = self.cfg
        b = cfg.batch
        fp8 = cfg.index_format == "fp8"
        kvc = None if kv is None else kv.contiguous()
        pos = self.positions.view(b, 1)
        from_table = isinstance(rope, str)
        if from_table and rope != "table":
            raise ValueError(f"step: rope must be a tuple of tables or 'table', got {rope!r}")
        if (compress is not None or from_table) and self.compressor is None:
            raise ValueError("step(compress=... / rope='table'): the layer was built without CompressorWeights")
        if from_table and compress is None:
            raise ValueError("step(rope='table'): the tables are gathered by the emission launch (compress=...)")
        if from_table and self._emit_prologue:
            if kvc is None or self.kv_norm_weight is None:
                raise ValueError("step(rope='table'): needs the kv projection and the layer's kv_norm_weight")
            if self._merged_emit:
                self._emit_scores(compress, kvc, q_idx.contiguous(), w)
                self._select_and_attend(q, (self.step_cos, self.step_sin), advance)
                return self.out if self.out_proj is None else self.out_proj(self.out)
            self._emit(compress, True, prologue=(kvc, q_idx.contiguous()))
            pos = self.positions.view(b, 1)
            if fp8:
                indexer.scores_fp8(self.q_codes, self.q_scales, w.view(b, 1, -1), self.k_codes, self.k_scales,
                                   compress_ratio=cfg.ratio, positions=pos, out=self.scores)
            else:
                indexer.scores_mxfp4(self.q_codes, self.q_e8m0, w.view(b, 1, -1), self.k_packed, self.k_e8m0,
                                     compress_ratio=cfg.ratio, positions=pos, out=self.scores)
            self._select_and_attend(q, (self.step_cos, self.step_sin), advance)
            return self.out if self.out_proj is None else self.out_proj(self.out)
        if compress is not None:
            self._emit(compress, from_table)
        if from_table:
            rope = (self.step_cos, self.step_sin, self.step_cos, self.step_sin)
        if rope is not None:
            return self._step_fused(q, kvc, q_idx, w, advance, rope)
        if fp8:
            # window append + indexer-query quantization + scores, one launch
            indexer.decode_fp8(q_idx, w.view(b, -1), self.k_codes, self.k_scales, compress_ratio=cfg.ratio,
                               positions=pos, out=self.scores, kv=kvc, win_cache=self.win, nope=cfg.nope,
                               rope=cfg.rope)
        elif cfg.index_dim == 128:
            # the same single launch for the MXFP4 index
            indexer.decode_mxfp4(q_idx, w.view(b, -1), self.k_packed, self.k_e8m0, compress_ratio=cfg.ratio,
                                 positions=pos, out=self.scores, kv=kvc, win_cache=self.win, nope=cfg.nope,
                                 rope=cfg.rope)
        else:
            # window append + indexer-query quantization (one launch), then scores
            qc = q_idx.contiguous()
            _lib.require_gpu(qc, *(() if kvc is None else (kvc,)))
            _lib.call("mzk_decode_prologue", _lib.ptr(kvc), _lib.dtype_code((qc if kvc is None else kvc).dtype),
                      0 if kvc is None else b, cfg.nope, cfg.rope, self.positions.data_ptr(), self.win.data_ptr(),
                      cfg.window, cfg.window, qc.data_ptr(), _lib.dtype_code(qc.dtype), b * cfg.index_heads,
                      cfg.index_dim, 1, self.q_codes.data_ptr(), None, self.q_e8m0.data_ptr(), _lib.stream_of(qc))
            indexer.scores_mxfp4(self.q_codes, self.q_e8m0, w.view(b, 1, -1), self.k_packed, self.k_e8m0,
                                 compress_ratio=cfg.ratio, positions=pos, out=self.scores)
        self._select_and_attend(q, None, advance)
        return self.out

    def _step_fused(self, q, kv, q_idx, w, advance, rope):
        cfg = self.cfg
        b = cfg.batch
        if kv is None or self.kv_norm_weight is None:
            raise ValueError("step(rope=...): needs the kv projection and the layer's kv_norm_weight")
        if cfg.index_dim != 128:
            raise ValueError(f"step(rope=...): the fused prologue needs index_dim 128, got {cfg.index_dim}")
        cos, sin, icos, isin = rope
        fp8 = cfg.index_format == "fp8"
        indexer.decode_fused(q_idx, w.view(b, -1), self.k_codes if fp8 else self.k_packed,
                             self.k_scales if fp8 else self.k_e8m0, fmt=cfg.index_format, compress_ratio=cfg.ratio,
                             positions=self.positions.view(b, 1), q_rope=(icos, isin), kv=kv,
                             kv_weight=self.kv_norm_weight, kv_eps=self.kv_norm_eps, kv_rope=(cos, sin),
                             win_cache=self.win, out=self.scores, nope=cfg.nope, rope=cfg.rope)
        self._select_and_attend(q, (cos, sin), advance)
        return self.out if self.out_proj is None else self.out_proj(self.out)

    @property
    def selects_in_attention(self) -> bool:
        """Whether the step's top-k runs inside the attention launch (``select_in_attention``,
        no branch overlap, at most 8192 keys and a top-2048, multiples of 4)."""
        cfg = self.cfg
        return (cfg.select_in_attention and not cfg.branch_overlap and cfg.max_groups <= 8192 and cfg.topk <= 2048
                and cfg.max_groups % 4 == 0 and cfg.topk % 4 == 0)

    def _select_and_attend(self, q, rope, advance=False):
        """Top-k, then the attention over [window ; dense ; top-k entries] with the sink, and
        with ``advance`` the positions' ``+= 1`` (in the merge launch).  With
        ``branch_overlap`` the window and dense branches run on the side stream while the
        top-k runs, each launch writing its own splits of the shared workspace, and one merge
        takes them all (the same softmax over the concatenated entries)."""
        cfg = self.cfg
        b = cfg.batch
        if self.selects_in_attention:
            csa2_attn.sparse_mqa_decode_select(q, self.positions, self.win, cfg.window, main_cache=self.main,
                                               scores=self.scores.view(b, cfg.max_groups), topk=cfg.topk,
                                               idx_out=self.idx, dense_cache=self.coarse,
                                               dense_ratio=max(cfg.coarse_ratio, 1), sinks=self.sinks,
                                               nsplit=cfg.nsplit, nope=cfg.nope, workspace=self.workspace,
                                               out=self.out, lse=self.lse, rope=rope, advance=advance)
            return
        if not cfg.branch_overlap:
            indexer.topk(self.scores.view(b, cfg.max_groups), cfg.topk, out=self.idx, workspace=self.topk_ws)
            csa2_attn.sparse_mqa_decode(q, self.positions, self.win, cfg.window, main_cache=self.main,
                                        groups=cfg.max_groups, indices=self.idx, dense_cache=self.coarse,
                                        dense_ratio=max(cfg.coarse_ratio, 1), sinks=self.sinks, nsplit=cfg.nsplit,
                                        nope=cfg.nope, workspace=self.workspace, out=self.out, lse=self.lse,
                                        rope=rope, advance=advance)
            return
        # the side stream reads q and the RoPE tables while the main stream runs on: they
        # must be the caller's own tensors, not temporaries the caching allocator could hand
        # to main-stream work before the side-stream launch has read them
        qc = q
        _lib.require_gpu(qc)
        if qc.dtype != torch.bfloat16 or qc.shape != (b, cfg.heads, cfg.dim) or not qc.is_contiguous():
            raise ValueError(f"step: q must be a contiguous bf16 [{b}, {cfg.heads}, {cfg.dim}] tensor")
        rc = rs = None
        if rope is not None:
            rc, rs = rope[0], rope[1]
            if not (rc.is_contiguous() and rs.is_contiguous()):
                raise ValueError("step(branch_overlap): the RoPE tables must be contiguous")
        total = self.nsplit_wd + cfg.nsplit
        ws = self.workspace
        wsb = ws.numel() * ws.element_size()
        rope_args = (_lib.ptr(rc), _lib.ptr(rs), cfg.rope if rope is not None else 0)
        coarse = self.coarse
        main = torch.cuda.current_stream(self.device)
        side = self._side
        side.wait_stream(main)  # the window append of this step is in the launch before
        with torch.cuda.stream(side):
            _lib.call("mzk_sparse_mqa_part", qc.data_ptr(), b, 1, cfg.heads, cfg.dim, 1, cfg.nope,
                      self.positions.data_ptr(), self.win.data_ptr(), cfg.window, cfg.window, cfg.window,
                      _lib.ptr(coarse), cfg.coarse_groups, cfg.coarse_groups, max(cfg.coarse_ratio, 1), None, 0, 0,
                      None, 0, 0, self.nsplit_wd, 0, total, ws.data_ptr(), wsb, *rope_args, side.cuda_stream)
        indexer.topk(self.scores.view(b, cfg.max_groups), cfg.topk, out=self.idx, workspace=self.topk_ws)
        _lib.call("mzk_sparse_mqa_part", qc.data_ptr(), b, 1, cfg.heads, cfg.dim, 1, cfg.nope,
                  self.positions.data_ptr(), None, 0, 0, 0, None, 0, 0, 1, self.main.data_ptr(), cfg.max_groups,
                  cfg.max_groups, self.idx.data_ptr(), cfg.topk, cfg.topk, cfg.nsplit, self.nsplit_wd, total,
                  ws.data_ptr(), wsb, *rope_args, main.cuda_stream)
        main.wait_stream(side)
        if rope is None:
            _lib.call("mzk_sparse_mqa_combine", ws.data_ptr(), b, 1, cfg.heads, cfg.dim, total, _lib.ptr(self.sinks),
                      self.out.data_ptr(), self.lse.data_ptr(), main.cuda_stream)
        else:
            _lib.call("mzk_sparse_mqa_combine_rope", ws.data_ptr(), b, 1, cfg.heads, cfg.dim, total,
                      _lib.ptr(self.sinks), rc.data_ptr(), rs.data_ptr(), cfg.rope, self.out.data_ptr(),
                      self.lse.data_ptr(), main.cuda_stream)
        if advance:
            self.positions.add_(1)

    def capture(self, q, kv, q_idx, w, advance: bool = False, warmup: int = 2,
                rope: tuple | str | None = None, compress: tuple | None = None,
                allow_stale_groups: bool = False) -> torch.cuda.CUDAGraph:
        """Record ``step`` into a HIP graph over static copies of the inputs; ``replay``
        then reruns it after the caller writes new inputs into ``static_inputs`` (q, kv,
        q_idx, w, then the ``rope`` tables when given as a tuple -- a replay that advances the
        positions needs the next position's tables written there too, which ``rope="table"``
        does on the device -- then the ``compress`` projections).

        ``advance=True`` needs the in-step emission (``compress``): without it a replay that
        completes a group would expose a cache slot nothing wrote.  ``allow_stale_groups``
        waives that for a caller whose caches already hold every group a replay can reach."""
        if advance and compress is None and not allow_stale_groups:
            raise ValueError("capture(advance=True) needs compress=(...) projections (in-step group emission); "
                             "pass allow_stale_groups=True if the caches already hold every reachable group")
        tabs = tuple(rope) if isinstance(rope, tuple) else ()
        comp = () if compress is None else tuple(compress)
        ins = (q, kv, q_idx, w) + tabs + comp
        self._static = tuple(None if t is None else t.clone() for t in ins)
        st = self._static
        nt = len(tabs)
        rope_arg = rope if isinstance(rope, str) else (st[4:4 + nt] if nt else None)
        comp_arg = st[4 + nt:] if comp else None
        run = lambda adv: self.step(*st[:4], advance=adv, rope=rope_arg, compress=comp_arg)  # noqa: E731
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        saved = self.positions.clone()
        saved_max = self._pos_max
        with torch.cuda.stream(s):
            for _ in range(warmup):
                run(False)
        torch.cuda.current_stream(self.device).wait_stream(s)
        self.positions.copy_(saved)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run(advance)
        self._pos_max = saved_max  # recording ran nothing
        self._graph = g
        self._graph_advances = advance
        return g

    @property
    def static_inputs(self):
        return self._static

    def replay(self) -> torch.Tensor:
        if self._graph_advances:
            self._check_table()
        self._graph.replay()
        if self._graph_advances and self._pos_max is not None:
            self._pos_max += 1
        return self.out
