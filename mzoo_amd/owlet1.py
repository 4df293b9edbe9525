"""Drop-in modules for mzoo's DeepSeek-V4.1 (owlet1) CSA2 attention on MI355X.

Same class names, constructor arguments, parameter names (``state_dict``-compatible) and
forward signatures as ``src/mzoo/archs/owlet1/{attention,cache,indexer,norm_rope}.py``:

* ``DeepseekV41Attention(config, layer_idx).forward(hidden_states, position_embeddings,
  attention_mask, past_key_values, shared, **kwargs) -> (out, None)``  (attention.py:74-236)
* ``DeepseekV41Compressor(config, layer_idx).forward(hidden_states, cache_layer)
  -> (latent | None, first_group_position)``                          (cache.py:127-172)
* ``DeepseekV41Indexer(config, layer_idx).forward(hidden_states, q_residual, latent,
  first_group_position, position_ids, cache_layer, shared) -> None``   (indexer.py:50-165)
* ``DeepseekV41CSACache(config)`` -- the KV-source cache layer         (cache.py:13-124)
* ``DeepseekV41RMSNorm``, ``DeepseekV41RotaryEmbedding``, ``apply_rotary_pos_emb``,
  ``DeepseekV41GroupedLinear``                                         (norm_rope.py, attention.py:20-39)
* ``sparse_attention_forward`` -- an attention interface with the signature of
  ``eager_attention_forward`` (attention.py:42-71), registered in transformers'
  ``ALL_ATTENTION_FUNCTIONS`` as ``"mzoo_amd_sparse"`` by ``register_attention_interface()``,
  so the reference's own module can run its attention here.

The projections (``wq_a``, ``wq_b``, ``wkv``, ``wo_a``, ``wo_b``, the compressor's and the
indexer's linears) are torch GEMMs (hipBLASLt); every per-token op runs in the HIP library:
RMSNorm, RoPE and its inverse, the FP8 / FP4 fake quantizers, the compressor's gated pooling,
the MXFP4 (or bf16) indexer scores with the group-causal mask, the top-k, the selection
formats and the sparse latent MQA with its sink.  There is no CPU path: CPU tensors raise.

The indexer publishes its selection as ``shared["topk_idx"]`` (int32 [B, S, k], ascending,
``-1`` = empty) and keeps ``shared["topk_bias"]`` (the reference's [B, 1, S, G] 0 / -inf bias)
available: a ``SharedState`` dict builds it on first access, a plain dict gets it at once.

Semantics kept from the reference: the window holds the last ``sliding_window`` tokens
(self included) and the mask is the model's sliding causal mask, so positions are the
running token count (``position_ids = past_seen + arange(S)``, decoder.py:285-288); the
compressed branch attends the groups the indexer kept; the top-k keeps ``min(k, G)``
entries, never a masked one, the lower index winning among equal scores (the reference's
``torch.topk`` leaves ties unspecified).  Attention runs in bf16 on MFMA with fp32 softmax
(the cached K = V entries are FP8 / FP4 fake-quantized, so exact in bf16); queries are
rounded to bf16.  Training (dropout, backward) is not supported.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F
from torch import nn
from transformers.cache_utils import DynamicSlidingWindowLayer

from . import _lib, csa2_attn, indexer as _idx, quant
from .rope import rope_inv_freq

_FMT_BF16 = csa2_attn.FMT_BF16


# ---- configuration ------------------------------------------------------------------------

@dataclass
class AttentionConfig:
    """The fields of ``DeepseekV41TextConfig`` (owlet1/config.py:226-296) these modules read.
    Any object with these attributes works (the reference's config included)."""
    hidden_size: int = 5120
    num_attention_heads: int = 64
    head_dim: int = 512
    qk_rope_head_dim: int = 64
    q_lora_rank: int = 1280
    o_groups: int = 8
    o_lora_rank: int = 1024
    rope_theta: float = 10000.0
    compress_rope_theta: float = 160000.0
    sliding_window: int = 128
    compress_ratios: list = field(default_factory=lambda: [4])
    kv_source_layer_ids: list = field(default_factory=lambda: [0])
    index_source_layer_ids: list = field(default_factory=lambda: [0])
    candidate_source_layer_id: int = -1
    candidate_topk_blocks: int = 2048
    candidate_block_size: int = 8
    index_n_heads: int = 32
    index_head_dim: int = 128
    index_topk: int = 512
    rms_norm_eps: float = 1e-20
    attention_dropout: float = 0.0
    _attn_implementation: str = "mzoo_amd_sparse"


def _rope_params(config, layer_type: str) -> tuple[float, float, dict | None]:
    """(theta, partial_rotary_factor, yarn) of a rope layer type ("main" / "compress"), from
    ``config.rope_parameters`` when present (owlet1/config.py:420-434), else from the flat
    fields.  ``yarn`` is None for the default RoPE, else the YaRN settings ``yarn_inv_freq``
    takes (owlet1/config.py:419-434: the reference applies YaRN to the compressed branches
    only and fixes its attention factor at 1.0 unless one is given)."""
    rp = getattr(config, "rope_parameters", None)
    if isinstance(rp, dict) and isinstance(rp.get(layer_type), dict):
        sub = rp[layer_type]
        kind = sub.get("rope_type", "default")
        yarn = None
        if kind == "yarn":
            orig = sub["original_max_position_embeddings"]
            factor = sub["factor"]
            if factor is None:
                factor = getattr(config, "max_position_embeddings") / orig
            yarn = dict(factor=float(factor), original_max_position_embeddings=orig,
                        beta_fast=sub.get("beta_fast") or 32, beta_slow=sub.get("beta_slow") or 1,
                        attention_factor=sub.get("attention_factor"), mscale=sub.get("mscale"),
                        mscale_all_dim=sub.get("mscale_all_dim"),
                        # read from the top level of rope_parameters, as the library the
                        # reference calls does (transformers' _compute_yarn_parameters)
                        truncate=rp.get("truncate", True))
        elif kind != "default":
            raise NotImplementedError(f"{layer_type} RoPE type {kind!r}: the default RoPE and YaRN are built")
        return float(sub["rope_theta"]), float(sub.get("partial_rotary_factor", 1.0)), yarn
    theta = config.compress_rope_theta if layer_type == "compress" else config.rope_theta
    return float(theta), config.qk_rope_head_dim / config.head_dim, None


# ---- norm / rope --------------------------------------------------------------------------

class DeepseekV41RMSNorm(nn.Module):
    """norm_rope.py:16-33 on the GPU (``mzk_rms_norm``): ``weight * dtype(h * rsqrt(mean(h^2)
    + eps))`` in fp32, summed in a fixed order."""

    def __init__(self, hidden_size, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        x = hidden_states
        _lib.require_gpu(x, self.weight)
        d = x.shape[-1]
        xc = x if x.stride(-1) == 1 and x.is_contiguous() else x.contiguous()
        w = self.weight.detach()
        out = torch.empty(x.shape, dtype=torch.promote_types(w.dtype, x.dtype), device=x.device)
        rows = xc.numel() // d
        _lib.call("mzk_rms_norm", xc.data_ptr(), _lib.dtype_code(x.dtype), rows, d, d, w.contiguous().data_ptr(),
                  _lib.dtype_code(w.dtype), float(self.variance_epsilon), out.data_ptr(),
                  _lib.dtype_code(out.dtype), _lib.stream_of(x))
        return out

    def extra_repr(self):
        return f"{tuple(self.weight.shape)}, eps={self.variance_epsilon}"


class DeepseekV41RotaryEmbedding(nn.Module):
    """norm_rope.py:48-124: per layer type ``inv_freq`` -- the default RoPE ``1 /
    theta^(2i/rd)``, or YaRN (``yarn_inv_freq``) where the config asks for it -- with ``rd =
    int(head_dim * partial_rotary_factor)``; ``forward`` returns cos / sin [B, S, rd/2] of
    ``position_ids`` times the type's attention factor, in ``x.dtype``."""

    def __init__(self, config, device=None):
        super().__init__()
        self.config = config
        self.layer_types = ["main", "compress"]
        self.attention_scaling = {}
        for lt in self.layer_types:
            theta, partial, yarn = _rope_params(config, lt)
            inv, scale = rope_inv_freq(theta, int(config.head_dim * partial), yarn)
            self.attention_scaling[lt] = scale
            self.register_buffer(f"{lt}_inv_freq", inv.to(device) if device is not None else inv, persistent=False)

    @torch.no_grad()
    def forward(self, x, position_ids, layer_type=None):
        inv = getattr(self, f"{layer_type}_inv_freq").float().to(x.device)
        scale = self.attention_scaling[layer_type]
        pos = position_ids.to(x.device).float()
        freqs = (inv[None, :, None].expand(pos.shape[0], -1, 1) @ pos[:, None, :]).transpose(1, 2)
        return (freqs.cos() * scale).to(dtype=x.dtype), (freqs.sin() * scale).to(dtype=x.dtype)


def apply_rotary_pos_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, inverse: bool = False):
    """norm_rope.py:126-145 on the GPU (``mzk_rope``): interleaved (even, odd) pairs of the
    trailing ``2 * cos.shape[-1]`` channels, fp32 math, ``inverse`` conjugates.  x [B, S, D]
    or [B, S, H, D]; cos / sin [B, S, rd/2]."""
    _lib.require_gpu(x)
    rd = cos.shape[-1] * 2
    d = x.shape[-1]
    heads = x.shape[2] if x.dim() == 4 else 1
    xc = x.contiguous()
    c = cos.float().contiguous()
    s = sin.float().contiguous()
    rows = xc.numel() // d
    if c.numel() * heads != rows * (rd // 2):
        raise ValueError(f"apply_rotary_pos_emb: cos/sin {tuple(cos.shape)} do not match x {tuple(x.shape)}")
    y = torch.empty_like(xc)
    _lib.call("mzk_rope", xc.data_ptr(), _lib.dtype_code(x.dtype), c.data_ptr(), s.data_ptr(), rows, d, rd, heads,
              int(bool(inverse)), y.data_ptr(), _lib.stream_of(x))
    return y


class DeepseekV41GroupedLinear(nn.Linear):
    """attention.py:20-39: block-diagonal projection of ``n_groups`` head groups (a batched
    GEMM; the weight is made contiguous as the batched product's right operand)."""

    def __init__(self, in_features_per_group: int, out_features: int, n_groups: int, bias: bool = False):
        super().__init__(in_features_per_group, out_features, bias=bias)
        self.n_groups = n_groups

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-2]
        hid = x.shape[-1]
        w = self.weight.view(self.n_groups, -1, hid).transpose(1, 2).contiguous()
        xg = x.reshape(-1, self.n_groups, hid).transpose(0, 1).contiguous()
        y = torch.bmm(xg, w).transpose(0, 1)
        return y.reshape(*lead, self.n_groups, -1)


def _fake_fp8(x, block_size=32):
    return quant._fake_quant_fp8_block(x, block_size)


def _fake_fp4(x, block_size, e4m3_scales=False):
    return quant._fake_quant_fp4_block(x, block_size, e4m3_scales=e4m3_scales)


# ---- the shared protocol ------------------------------------------------------------------

class SharedState(dict):
    """The per-forward ``shared`` dict, with ``"topk_bias"`` built from ``"topk_idx"`` only
    when a consumer reads it (the reference's reuse-mode layers, owlet1/attention.py:171)."""

    def _materialize(self):
        if dict.__contains__(self, "topk_bias") or not dict.__contains__(self, "_topk_bias_src"):
            return
        idx, groups = dict.pop(self, "_topk_bias_src")
        dict.__setitem__(self, "topk_bias", _topk_bias(idx, groups))

    def __getitem__(self, key):
        if key == "topk_bias":
            self._materialize()
        return dict.__getitem__(self, key)

    def get(self, key, default=None):
        if key == "topk_bias":
            self._materialize()
        return dict.get(self, key, default)

    def __contains__(self, key):
        if key == "topk_bias":
            return dict.__contains__(self, "topk_bias") or dict.__contains__(self, "_topk_bias_src")
        return dict.__contains__(self, key)


def _topk_bias(idx: torch.Tensor, groups: int) -> torch.Tensor:
    """indices int32 [B, S, k] -> the reference's bias [B, 1, S, G] fp32 (0 kept, -inf not)."""
    b, s, k = idx.shape
    bias = torch.empty(b, 1, s, groups, dtype=torch.float32, device=idx.device)
    _lib.call("mzk_topk_bias", idx.data_ptr(), b * s, k, k, groups, bias.data_ptr(), groups, _lib.stream_of(idx))
    return bias


def _publish_selection(shared: dict, idx: torch.Tensor, groups: int) -> None:
    shared["topk_idx"] = idx
    shared["_topk_groups"] = groups
    if isinstance(shared, SharedState):
        dict.pop(shared, "topk_bias", None)
        dict.__setitem__(shared, "_topk_bias_src", (idx, groups))
    else:
        shared["topk_bias"] = _topk_bias(idx, groups)


def _mask_to_indices(mask: torch.Tensor, cap: int) -> torch.Tensor:
    """additive mask [R, T] (0 visible; -inf or the dtype's lowest value masked) -> int32
    [R, cap] visible columns ascending, -1 after; raises for other values or overflow."""
    r, t = mask.shape
    m = mask if mask.stride(-1) == 1 else mask.contiguous()
    idx = torch.empty(r, cap, dtype=torch.int32, device=mask.device)
    counts = torch.empty(r, dtype=torch.int32, device=mask.device)
    flags = torch.zeros(1, dtype=torch.int32, device=mask.device)
    _lib.call("mzk_mask_to_indices", m.data_ptr(), _lib.dtype_code(m.dtype), r, t, m.stride(0), cap, idx.data_ptr(),
              counts.data_ptr(), flags.data_ptr(), _lib.stream_of(mask))
    f = int(flags.item())
    if f & 1:
        raise NotImplementedError("sparse attention: the mask holds values other than 0 / -inf / the dtype minimum")
    if f & 2:
        raise ValueError(f"sparse attention: a row has more than {cap} visible columns")
    return idx


# ---- the cache layer ----------------------------------------------------------------------

class _Growing:
    """An append-only [B, n, ...] tensor with amortized O(1) appends (capacity doubling)."""

    def __init__(self):
        self.buf = None
        self.n = 0

    def append(self, x: torch.Tensor) -> torch.Tensor:
        need = self.n + x.shape[1]
        if self.buf is None or need > self.buf.shape[1] or self.buf.shape[0] != x.shape[0] \
                or self.buf.shape[2:] != x.shape[2:] or self.buf.dtype != x.dtype:
            cap = max(need, 2 * (self.buf.shape[1] if self.buf is not None else 0), 16)
            nb = torch.empty(x.shape[0], cap, *x.shape[2:], dtype=x.dtype, device=x.device)
            if self.buf is not None and self.n:
                nb[:, :self.n] = self.buf[:, :self.n]
            self.buf = nb
        self.buf[:, self.n:need] = x
        self.n = need
        return self.view()

    def view(self):
        return None if self.buf is None else self.buf[:, :self.n]

    def reindex(self, fn):
        if self.buf is not None:
            v = fn(self.buf[:, :self.n])
            self.buf, self.n = v.contiguous(), v.shape[1]


class DeepseekV41CSACache(DynamicSlidingWindowLayer):
    """Cache layer of a KV-source layer (owlet1/cache.py:13-124): the sliding window of K = V
    entries (the last ``sliding_window - 1``), the partial group carried across calls, the
    running compressed latents and indexer keys, and the group count.  The running caches
    grow in place (``compressed_kv[...]`` are views of them), so a decode step appends one
    entry instead of copying the cache; the indexer keys are also kept in the packed MXFP4
    form the score kernel reads (``packed_index_k``)."""

    _layer_type = "shared_compressed_attention"

    def __init__(self, config, **kwargs):
        super().__init__(sliding_window=config.sliding_window)
        self.buffer_kv: dict = {"compressor": None}
        self.buffer_gate: dict = {"compressor": None}
        self._store = {"compressor": _Growing(), "indexer": _Growing()}
        self._packed = (_Growing(), _Growing())
        self._mirror = _Growing()  # bf16 copy of the compressed latents (a non-bf16 model)
        self.entry_count: dict = {"compressor": 0}

    @property
    def compressed_kv(self) -> dict:
        return {k: (None if g.buf is None else g.view().unsqueeze(1)) for k, g in self._store.items()}

    def compressed_bf16(self):
        """[B, G, D] bf16 view of the compressed latents, the attention kernel's entry
        format: the running cache itself for a bf16 model, else its bf16 mirror, appended as
        groups are emitted (the fake-quantized latents are exact in bf16)."""
        st = self._store["compressor"]
        if st.buf is None:
            return None
        return st.view() if st.buf.dtype == torch.bfloat16 else self._mirror.view()

    def packed_index_k(self):
        """(e2m1 codes [B, G, Di/2], e8m0 [B, G, Di/32]) of the indexer keys, or None."""
        p, e = self._packed
        return None if p.buf is None else (p.view(), e.view())

    def _reindex(self, fn):
        for g in (*self._store.values(), *self._packed, self._mirror):
            g.reindex(fn)
        for attr in ("buffer_kv", "buffer_gate"):
            buf = getattr(self, attr)
            for name, t in buf.items():
                if t is not None:
                    buf[name] = fn(t)

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        super().reorder_cache(beam_idx)
        self._reindex(lambda t: t.index_select(0, beam_idx.to(t.device)))

    def batch_repeat_interleave(self, repeats: int) -> None:
        super().batch_repeat_interleave(repeats)
        self._reindex(lambda t: t.repeat_interleave(repeats, dim=0))

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        super().batch_select_indices(indices)
        self._reindex(lambda t: t[indices, ...])

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """K = V sliding window: returns every entry the new queries can see (the cached
        ``sliding_window - 1`` plus the new ones) and keeps the last ``sliding_window - 1``."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
            self.values = self.keys
        self.cumulative_length += key_states.shape[-2]
        full = torch.cat([self.keys, key_states], dim=-2)
        self.keys = full[:, :, max(0, full.shape[-2] - (self.sliding_window - 1)):, :]
        self.values = self.keys
        return full, full

    def store_compression_weights(self, name: str, kv: torch.Tensor, gate, compress_ratio: int):
        """Prepend the carried partial group, split off the group-aligned prefix, carry the
        rest; returns (chunk_kv, chunk_gate, position of the chunk's first token)."""
        first = self.entry_count[name] * compress_ratio
        carried = self.buffer_kv[name]
        if carried is not None and carried.shape[1]:
            kv = torch.cat([carried, kv], 1)
            gate = None if gate is None else torch.cat([self.buffer_gate[name], gate], 1)
        cut = kv.shape[1] - kv.shape[1] % compress_ratio
        self.buffer_kv[name] = kv[:, cut:]
        self.buffer_gate[name] = None if gate is None else gate[:, cut:]
        return kv[:, :cut], (None if gate is None else gate[:, :cut]), first

    def update_compressor_states(self, name: str, compressed: torch.Tensor) -> torch.Tensor:
        """Append entries [B, 1, n, D] to the running cache ``name``; returns it [B, 1, G, D]."""
        if compressed.shape[2] > 0 or self._store[name].buf is None:
            self._store[name].append(compressed[:, 0])
            if name == "compressor" and compressed.dtype != torch.bfloat16:
                self._mirror.append(compressed[:, 0].to(torch.bfloat16))
        if name == "compressor":
            self.entry_count[name] += compressed.shape[2]
        return self._store[name].view().unsqueeze(1)

    def append_packed_index_k(self, codes: torch.Tensor, e8m0: torch.Tensor) -> None:
        self._packed[0].append(codes)
        self._packed[1].append(e8m0)


# ---- compressor ---------------------------------------------------------------------------

class DeepseekV41Compressor(nn.Module):
    """cache.py:127-172: pools ``compress_ratio`` tokens into one latent with a softmax gate
    (fp32 projections, the pooling and RMSNorm in one ``mzk_compress`` launch); returns the
    pre-RoPE latents of the groups completed in this call and the first one's position."""

    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.compress_ratio = config.compress_ratios[layer_idx]
        self.head_dim = config.head_dim
        self.wkv = nn.Linear(config.hidden_size, self.head_dim, bias=False)
        self.wgate = nn.Linear(config.hidden_size, self.head_dim, bias=False) if self.compress_ratio > 1 else None
        self.norm = DeepseekV41RMSNorm(self.head_dim, eps=config.rms_norm_eps)

    def forward(self, hidden_states: torch.Tensor, cache_layer):
        if self.wgate is None:
            latent = self.norm(self.wkv(hidden_states))
            return latent, 0 if cache_layer is None else cache_layer.entry_count["compressor"]
        r = self.compress_ratio
        x32 = hidden_states.float()
        kv = F.linear(x32, self.wkv.weight.float())
        gate = F.linear(x32, self.wgate.weight.float())
        if cache_layer is None:
            cut = kv.shape[1] - kv.shape[1] % r
            kv, gate, first = kv[:, :cut], gate[:, :cut], 0
        else:
            kv, gate, first = cache_layer.store_compression_weights("compressor", kv, gate, r)
        if kv.shape[1] == 0:
            return None, first
        w = self.norm.weight.detach()
        if w.dtype != hidden_states.dtype:
            raise ValueError("DeepseekV41Compressor: the norm weight and the hidden states must share a dtype")
        b, t, d = kv.shape
        out = torch.empty(b, t // r, d, dtype=hidden_states.dtype, device=kv.device)
        kvc, gc = kv.contiguous(), gate.contiguous()
        _lib.call("mzk_compress", kvc.data_ptr(), gc.data_ptr(), b, t // r, r, d, t, w.contiguous().data_ptr(),
                  _lib.dtype_code(w.dtype), float(self.norm.variance_epsilon), out.data_ptr(),
                  _lib.dtype_code(out.dtype), _lib.stream_of(kv))
        return out, first


# ---- indexer ------------------------------------------------------------------------------

class DeepseekV41Indexer(nn.Module):
    """indexer.py:50-165: publishes the keys of the groups completed in this call (``k_norm(
    wk(latent))``, compress RoPE at the groups' positions, MXFP4 fake quant), scores the
    queries against every published key on MFMA (``Di^-0.5 * sum_h w_h relu(q_h . k)``, the
    group-causal mask inside the kernel) and keeps the top ``index_topk`` per query."""

    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.layer_idx = layer_idx
        self.owns_k = layer_idx in config.kv_source_layer_ids
        self.compress_ratio = config.compress_ratios[layer_idx]
        self.is_candidate_source = layer_idx == config.candidate_source_layer_id
        self.uses_candidates = 0 <= config.candidate_source_layer_id < layer_idx
        self.candidate_topk_blocks = config.candidate_topk_blocks
        self.candidate_block_size = config.candidate_block_size
        self.num_heads = config.index_n_heads
        self.head_dim = config.index_head_dim
        self.index_topk = config.index_topk
        self.softmax_scale = self.head_dim ** -0.5
        self.heads_scaling = self.num_heads ** -0.5
        self.wq_b = nn.Linear(config.q_lora_rank, self.num_heads * self.head_dim, bias=False)
        self.weights_proj = nn.Linear(config.hidden_size, self.num_heads, bias=False)
        self.rotary_emb = DeepseekV41RotaryEmbedding(config)
        if self.owns_k:
            self.wk = nn.Linear(config.head_dim, self.head_dim, bias=False)
            self.k_norm = DeepseekV41RMSNorm(self.head_dim, eps=config.rms_norm_eps)

    def _packed_ok(self) -> bool:
        return self.head_dim % 64 == 0 and self.num_heads <= 64

    def forward(self, hidden_states, q_residual, latent, first_group_position, position_ids, cache_layer, shared):
        b, s, _ = hidden_states.shape
        r = self.compress_ratio
        packed = self._packed_ok()
        if self.owns_k:
            if latent is not None:
                k = self.k_norm(self.wk(latent))
                gpos = first_group_position + r * torch.arange(latent.shape[1], device=k.device)
                cos, sin = self.rotary_emb(k, position_ids=gpos.unsqueeze(0).expand(b, -1), layer_type="compress")
                k = _fake_fp4(apply_rotary_pos_emb(k, cos, sin), 32)
                pk = quant.quant_mxfp4(k) if packed else None
                if cache_layer is not None:
                    cache_layer.update_compressor_states("indexer", k.unsqueeze(1))
                    if packed and hasattr(cache_layer, "append_packed_index_k"):
                        cache_layer.append_packed_index_k(*pk)
                else:
                    prev = shared.get("index_k")
                    shared["index_k"] = k.unsqueeze(1) if prev is None else torch.cat([prev, k.unsqueeze(1)], 2)
                    if packed:
                        pp = shared.get("index_k_packed")
                        shared["index_k_packed"] = pk if pp is None else tuple(
                            torch.cat([a, c], 1) for a, c in zip(pp, pk))
            if cache_layer is not None:
                shared["index_k"] = cache_layer.compressed_kv["indexer"]
                if packed and hasattr(cache_layer, "packed_index_k"):
                    shared["index_k_packed"] = cache_layer.packed_index_k()
        index_k = shared.get("index_k")
        g = 0 if index_k is None else index_k.shape[2]
        if g == 0:
            return

        cos_q, sin_q = self.rotary_emb(hidden_states, position_ids=position_ids, layer_type="compress")
        q = self.wq_b(q_residual).view(b, s, self.num_heads, self.head_dim)
        q = apply_rotary_pos_emb(q, cos_q, sin_q)
        w = (self.weights_proj(hidden_states).float() * self.heads_scaling).contiguous()
        pos = position_ids.to(device=q.device, dtype=torch.int64).expand(b, s).contiguous()
        scores = torch.empty(b, s, g, dtype=torch.float32, device=q.device)
        if packed:
            kp = shared.get("index_k_packed")
            if kp is None or kp[0].shape[1] != g:
                kp = quant.quant_mxfp4(index_k[:, 0])
            qp, qe = quant.quant_mxfp4(q)                                 # _fake_quant_fp4_block(q, 32), packed
            kc, ke = kp
            # the running caches are views of larger buffers: keys are rows of Di/2 (Di/32)
            # bytes, batches `stride(0)` apart, read in place when both share one key stride
            kbs = kc.stride(0) // (self.head_dim // 2)
            if not (kc.stride(2) == 1 and kc.stride(1) == self.head_dim // 2 and ke.stride(2) == 1
                    and ke.stride(1) == self.head_dim // 32 and ke.stride(0) // (self.head_dim // 32) == kbs):
                kc, ke = kc.contiguous(), ke.contiguous()
                kbs = g
            _lib.call("mzk_indexer_scores_mxfp4", qp.data_ptr(), qe.data_ptr(), w.data_ptr(), kc.data_ptr(),
                      ke.data_ptr(), b, s, self.num_heads, self.head_dim, g, kbs, pos.data_ptr(), r,
                      scores.data_ptr(), g, _lib.stream_of(q))
        else:
            # fake-quantized values are exact in bf16 (an e2m1 value times a power of two)
            qv = _fake_fp4(q, 32).to(torch.bfloat16).contiguous()
            kv = index_k[:, 0].to(torch.bfloat16).contiguous()
            _lib.call("mzk_indexer_scores_bf16", qv.data_ptr(), w.data_ptr(), kv.data_ptr(), b, s, self.num_heads,
                      self.head_dim, g, g, pos.data_ptr(), r, scores.data_ptr(), g, _lib.stream_of(q))

        if self.is_candidate_source:
            lens = ((pos + 1) // r).unsqueeze(-1)
            shared["candidates"] = _idx.select_candidate_blocks(scores, lens, self.candidate_topk_blocks,
                                                                 self.candidate_block_size)
        elif self.uses_candidates and shared.get("candidates") is not None:
            scores = scores.masked_fill(~shared["candidates"], float("-inf"))

        k_eff = min(self.index_topk, g)
        idx = _idx.topk(scores, k_eff)                                    # [B, S, k] int32 ascending, -1 pad
        _publish_selection(shared, idx, g)


# ---- attention ----------------------------------------------------------------------------

# keys of `shared` that belong to one group: a KV-source layer without a cache drops them
# before it opens its group, so a later group (possibly at another ratio) does not append to
# an earlier group's entries (archs/dsv4/modeling_deepseek_v41.py:722-732; the owlet1 module
# lacks the reset, archs/owlet1/GAPS.md item 2)
_GROUP_KEYS = ("compress_kv", "index_k", "index_k_packed", "topk_bias", "_topk_bias_src", "topk_idx",
               "_topk_groups", "candidates", "_compress_kv_bf16")


def _entries(x: torch.Tensor) -> tuple[torch.Tensor, int]:
    """[B, T, D] entries -> (bf16 [B, >= T, D] rows read in place when possible, entries
    between batches)."""
    d = x.shape[-1]
    if x.dtype == torch.bfloat16 and x.stride(-1) == 1 and x.stride(1) == d and x.stride(0) % d == 0 \
            and x.data_ptr() % 16 == 0:
        return x, x.stride(0) // d
    y = x.to(torch.bfloat16).contiguous()
    return y, y.shape[1]


def _compressed_bf16(shared: dict):
    """The group's compressed latents as bf16 [B, G, D] (converted once per forward, or the
    cache layer's persistent mirror its KV source published)."""
    src = shared.get("compress_kv")
    if src is None or src.shape[2] == 0:
        return None
    hit = shared.get("_compress_kv_bf16")
    if hit is not None and hit[0] is src:
        return hit[1]
    bf = src[:, 0].to(torch.bfloat16).contiguous()
    shared["_compress_kv_bf16"] = (src, bf)
    return bf


def _nsplit(rows: int) -> int:
    return 1 if rows >= 128 else max(1, min(16, 256 // max(rows, 1)))


def _sparse_attend(q: torch.Tensor, sinks: torch.Tensor, *, window=None, parts=()) -> torch.Tensor:
    """q [B, S, H, D] (any float dtype) -> bf16 [B, S, H, D] on ``mzk_sparse_mqa``, one softmax
    (with the sink) over every source:

    * ``window = (entries [B, T, D], rel_pos int64 [B*S], W)``: row r sees entries
      rel_pos[r]-W+1 .. rel_pos[r] of its batch (the kernel's linear window source);
    * ``parts = [(entries [B, T, D], idx int32 [B*S, k]), ...]``: row r sees entries
      idx[r, :] (-1 = none) -- at most one part beside a window; two parts without a window
      run as two partial launches into one workspace and one merge."""
    b, s, h, d = q.shape
    qb = q.to(torch.bfloat16).contiguous()
    out = torch.empty(b, s, h, d, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(b, h, s, dtype=torch.float32, device=q.device)
    rows = b * s
    dev = q.device
    parts = [(e, i) for e, i in parts if e is not None and i is not None and i.shape[-1] > 0 and e.shape[1] > 0]
    if window is not None:
        win, win_stride = _entries(window[0])
        pos, w = window[1], window[2]
    else:
        win, win_stride, w = None, 0, 0
        pos = torch.full((rows,), -1, dtype=torch.int64, device=dev)
    if window is not None and len(parts) > 1:
        raise ValueError("sparse attention: at most one indexed source beside the window")
    prepared = []
    for e, i in parts:
        e2, est = _entries(e)
        ic = i.reshape(rows, -1).to(torch.int32).contiguous()
        prepared.append((e2, est, e.shape[1], ic))
    if window is None and not prepared:
        out.zero_()                                   # nothing visible: the sink takes all mass
        return out
    if len(prepared) <= 1:
        ns = _nsplit(rows)
        ws = csa2_attn.new_workspace(rows, h, d, ns, dev) if ns > 1 else None
        e2, est, g, ic = prepared[0] if prepared else (None, 0, 0, None)
        k = 0 if ic is None else ic.shape[1]
        _lib.call("mzk_sparse_mqa", qb.data_ptr(), b, s, h, d, _FMT_BF16, d, pos.data_ptr(), _lib.ptr(win), win_stride,
                  0, w, None, 0, 0, 1, _lib.ptr(e2), est, g, _lib.ptr(ic), k, k, sinks.data_ptr(), ns, _lib.ptr(ws),
                  0 if ws is None else ws.numel() * ws.element_size(), out.data_ptr(), lse.data_ptr(),
                  _lib.stream_of(q))
        return out
    ns = max(1, _nsplit(rows) // len(prepared))
    total = ns * len(prepared)
    ws = csa2_attn.new_workspace(rows, h, d, total, dev)
    for j, (e2, est, g, ic) in enumerate(prepared):
        k = ic.shape[1]
        _lib.call("mzk_sparse_mqa_part", qb.data_ptr(), b, s, h, d, _FMT_BF16, d, pos.data_ptr(), None, 0, 0, 0, None, 0,
                  0, 1, e2.data_ptr(), est, g, ic.data_ptr(), k, k, ns, j * ns, total, ws.data_ptr(),
                  ws.numel() * ws.element_size(), None, None, 0, _lib.stream_of(q))
    _lib.call("mzk_sparse_mqa_combine", ws.data_ptr(), b, s, h, d, total, sinks.data_ptr(), out.data_ptr(),
              lse.data_ptr(), _lib.stream_of(q))
    return out


def _window_lists(shared: dict, attention_mask: torch.Tensor, b: int, s: int, t: int, window: int) -> torch.Tensor:
    """The visible window columns of the model's mask [B or 1, 1, S, >= T] as int32 index
    lists [B*S, cap] (ascending, -1 after).  The layers of a forward receive the same mask
    and the same window length, so the lists are built once per forward."""
    hit = shared.get("_window_lists")
    if hit is not None and hit[0] is attention_mask and hit[1] == t:
        return hit[2]
    m = attention_mask
    if m.dim() != 4 or m.shape[-2] != s or m.shape[-1] != t:
        raise ValueError(f"DeepseekV41Attention: attention_mask {tuple(m.shape)} does not cover the {s} queries "
                         f"x {t} window entries of this call")
    if m.dtype == torch.bool:
        m = torch.zeros(m.shape, dtype=torch.float32, device=m.device).masked_fill_(~m, float("-inf"))
    m = m.expand(b, 1, s, t).reshape(b * s, t)
    cap = min(t, window)
    try:
        lists = _mask_to_indices(m, cap)
    except ValueError:                                # more than `window` visible: not a sliding mask
        lists = _mask_to_indices(m, t)
    shared["_window_lists"] = (attention_mask, t, lists)
    return lists


class DeepseekV41Attention(nn.Module):
    """attention.py:74-236: latent shared-KV attention over the sliding window and, for a
    layer with a compressed branch, the compressed entries its group's indexer selected."""

    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.compress_ratio = config.compress_ratios[layer_idx]
        self.num_heads = config.num_attention_heads
        self.num_key_value_groups = config.num_attention_heads
        self.head_dim = config.head_dim
        self.rope_layer_type = "compress" if self.compress_ratio else "main"
        self.sliding_window = config.sliding_window
        self.attention_dropout = config.attention_dropout
        self.is_causal = True
        self.scaling = self.head_dim ** -0.5

        self.wq_a = nn.Linear(config.hidden_size, config.q_lora_rank, bias=False)
        self.q_norm = DeepseekV41RMSNorm(config.q_lora_rank, eps=config.rms_norm_eps)
        self.wq_b = nn.Linear(config.q_lora_rank, self.num_heads * self.head_dim, bias=False)
        self.wkv = nn.Linear(config.hidden_size, self.head_dim, bias=False)
        self.kv_norm = DeepseekV41RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.wo_a = DeepseekV41GroupedLinear(self.num_heads * self.head_dim // config.o_groups,
                                             config.o_groups * config.o_lora_rank, config.o_groups)
        self.wo_b = nn.Linear(config.o_groups * config.o_lora_rank, config.hidden_size, bias=False)
        self.attn_sink = nn.Parameter(torch.empty(self.num_heads))

        self.is_kv_source = layer_idx in config.kv_source_layer_ids
        self.is_index_source = layer_idx in config.index_source_layer_ids
        self.compressor = DeepseekV41Compressor(config, layer_idx) if self.is_kv_source else None
        self.indexer = DeepseekV41Indexer(config, layer_idx) if self.is_index_source else None
        self.compress_rotary = DeepseekV41RotaryEmbedding(config) if self.is_kv_source else None

    def forward(self, hidden_states, position_embeddings, attention_mask, past_key_values, shared, **kwargs):
        """attention.py:129-236.  The window is what the model's mask keeps of this call's
        window entries (the cached ``sliding_window - 1`` and the new ones): a 4-D additive
        (0 / -inf / the dtype's lowest value) or bool mask is turned into index lists, so
        padding and any other 0 / -inf pattern are honoured exactly; other mask values raise
        NotImplementedError.  Without a mask (an attention implementation that builds none)
        row t sees the ``sliding_window`` entries ending at itself in token order.  The
        compressed branch attends the entries the group's indexer selected, or none when no
        index source ran in this forward (attention.py:202-214)."""
        if self.training and self.attention_dropout > 0:
            raise NotImplementedError("DeepseekV41Attention (mzoo_amd): inference only, no attention dropout")
        position_ids = kwargs["position_ids"]
        batch, seq_len, _ = hidden_states.shape
        cos, sin = position_embeddings[self.rope_layer_type]

        q_residual = self.q_norm(self.wq_a(hidden_states))
        q = self.wq_b(q_residual).view(batch, seq_len, self.num_heads, self.head_dim)
        q = apply_rotary_pos_emb(q, cos, sin)                                 # [B, S, H, D]
        kv = self.kv_norm(self.wkv(hidden_states))
        kv = _fake_fp8(apply_rotary_pos_emb(kv, cos, sin), 32)                # attention.py:149-154
        if past_key_values is not None:
            full = past_key_values.update(kv.unsqueeze(1), kv.unsqueeze(1), self.layer_idx)[0][:, 0]
        else:
            full = kv

        idx = comp = None
        if self.compress_ratio:
            cache_layer = past_key_values.layers[self.layer_idx] if past_key_values is not None else None
            if self.is_kv_source and cache_layer is None:
                for key in _GROUP_KEYS:
                    shared.pop(key, None)
            latent, first_group_position = (None, 0)
            if self.is_kv_source:
                latent, first_group_position = self.compressor(hidden_states, cache_layer)
            if self.is_index_source:
                self.indexer(hidden_states, q_residual, latent, first_group_position, position_ids, cache_layer,
                             shared)
            if latent is not None:
                gpos = first_group_position + self.compress_ratio * torch.arange(latent.shape[1],
                                                                                  device=latent.device)
                cos_c, sin_c = self.compress_rotary(latent, position_ids=gpos.unsqueeze(0).expand(batch, -1),
                                                    layer_type="compress")
                rotated = _fake_fp4(apply_rotary_pos_emb(latent, cos_c, sin_c), 16, e4m3_scales=True).unsqueeze(1)
                if cache_layer is not None:
                    cache_layer.update_compressor_states("compressor", rotated)
                else:
                    prev = shared.get("compress_kv")
                    shared["compress_kv"] = rotated if prev is None else torch.cat([prev, rotated], dim=2)
            if self.is_kv_source and cache_layer is not None:
                running = cache_layer.compressed_kv["compressor"]
                shared["compress_kv"] = running
                if hasattr(cache_layer, "compressed_bf16") and running is not None and running.shape[2]:
                    shared["_compress_kv_bf16"] = (running, cache_layer.compressed_bf16())
            comp = _compressed_bf16(shared)
            if comp is not None:
                g = comp.shape[1]
                if "topk_idx" in shared:
                    idx = shared["topk_idx"]
                    if shared.get("_topk_groups", g) != g:
                        raise ValueError(f"DeepseekV41Attention layer {self.layer_idx}: the selection published in "
                                         f"this forward covers {shared.get('_topk_groups')} compressed entries, the "
                                         f"group's cache holds {g}")
                elif shared.get("topk_bias") is not None:                    # a reference indexer published
                    bias = shared["topk_bias"]
                    if bias.shape[-1] != g:
                        raise ValueError(f"DeepseekV41Attention layer {self.layer_idx}: topk_bias covers "
                                         f"{bias.shape[-1]} compressed entries, the group's cache holds {g}")
                    idx = _mask_to_indices(bias.reshape(-1, g), min(self.config.index_topk, g))
                if idx is None:
                    comp = None                                              # no index source: none attended

        sinks = self.attn_sink.detach().float().contiguous()
        t = full.shape[1]
        if isinstance(attention_mask, torch.Tensor):
            lists = _window_lists(shared, attention_mask, batch, seq_len, t, self.sliding_window)
            o = _sparse_attend(q, sinks, parts=[(full, lists), (comp, idx)])
        else:
            rel = (t - seq_len + torch.arange(seq_len, device=q.device, dtype=torch.int64)).repeat(batch)
            o = _sparse_attend(q, sinks, window=(full, rel, self.sliding_window), parts=[(comp, idx)])
        o = apply_rotary_pos_emb(o.to(hidden_states.dtype), cos, sin, inverse=True)  # attention.py:231-233
        grouped = o.reshape(batch, seq_len, self.config.o_groups, -1)
        output = self.wo_b(self.wo_a(grouped).flatten(2))
        return output, None


# ---- the attention interface --------------------------------------------------------------

def sparse_attention_forward(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
    """``eager_attention_forward`` (owlet1/attention.py:42-71) on the sparse kernel: query
    [B, H, S, D], key == value [B, 1, T, D], attention_mask [B, 1, S, T] additive (0 kept,
    -inf / the dtype's lowest value masked -- the sliding causal mask extended by the
    indexer's ``topk_bias``).  Each row's visible columns become an index list and the kernel
    attends exactly those, with ``module.attn_sink`` in the denominator.  Returns
    ([B, S, H, D] in the query's dtype, None).  ``scaling`` must be ``D^-0.5``."""
    if dropout:
        raise NotImplementedError("sparse_attention_forward: inference only (dropout must be 0)")
    if key is not value and not torch.equal(key, value):
        raise NotImplementedError("sparse_attention_forward: shared-latent attention needs key == value")
    b, h, s, d = query.shape
    if abs(scaling - d ** -0.5) > 1e-6 * d ** -0.5:
        raise NotImplementedError(f"sparse_attention_forward: scaling must be head_dim^-0.5, got {scaling}")
    t = key.shape[2]
    if attention_mask is None:
        raise NotImplementedError("sparse_attention_forward: needs the additive mask")
    mask = attention_mask.expand(b, 1, s, t).reshape(b * s, t)
    cfg = module.config
    cap = min(t, cfg.sliding_window + (getattr(cfg, "index_topk", 0) if module.compress_ratio else 0))
    idx = _mask_to_indices(mask, cap).view(b, s, cap)
    q = query.transpose(1, 2)
    o = _sparse_attend(q, module.attn_sink.detach().float().contiguous(), parts=[(key[:, 0], idx)])
    return o.to(query.dtype), None


def register_attention_interface(name: str = "mzoo_amd_sparse") -> str:
    """Register ``sparse_attention_forward`` in transformers' ``ALL_ATTENTION_FUNCTIONS`` so a
    model whose ``config._attn_implementation`` is ``name`` runs its attention here."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    ALL_ATTENTION_FUNCTIONS.register(name, sparse_attention_forward)
    return name
