"""CPU: pin the module-composition oracle (oracle/model.py) against the reference's own
``DeepseekV41Attention`` run on the CPU (tests/golden/module_fixture.npz, written by
tests/golden/make_module_fixture.py).

Checked for the small configuration (full outputs) and BASELINE config 1 (B1 S1024, sampled
output rows, every row's selection):

* the layer output without a cache and with a cache fed in chunks (two prefill chunks that
  end mid-group, then one-token decode steps), with the reference's selection imposed --
  the reference's ``torch.topk`` breaks ties in a shape-dependent order;
* the oracle's own top-k equals the reference's selection wherever the reference's
  selection is not decided by a tie (ReLU gives many exact zero scores), and where they
  differ every differing entry scores exactly the k-th score;
* the published indexer keys and compressed latents, the window, the group count and the
  carried partial group after the chunked run.
"""

import pathlib
import sys

import numpy as np
import pytest

from oracle import model as M

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))
import module_spec as spec  # noqa: E402

FIX = np.load(HERE / "golden" / "module_fixture.npz")


def _cfg(c):
    return dict(c, rms_norm_eps=spec.RMS_NORM_EPS, compress_rope_theta=spec.COMPRESS_ROPE_THETA)


def _sel(name, key, groups):
    return np.unpackbits(FIX[f"{name}/{key}"], axis=-1)[..., :groups].astype(bool)


def _rows(name, out):
    if name == "config1":
        return out[:, FIX["config1/sample_rows"]]
    return out


def _assert_close(got, want, what, rtol=2e-5):
    err = np.abs(got - want).max()
    scale = np.abs(want).max()
    assert err <= rtol * scale, f"{what}: max err {err:.3e} vs scale {scale:.3e}"


def _ties_only(sel_ref, sel_mine, scores, what):
    """Rows where the two selections differ: every differing entry has the k-th score."""
    rows = np.argwhere((sel_ref != sel_mine).any(-1))
    for b, s in rows:
        diff = np.nonzero(sel_ref[b, s] != sel_mine[b, s])[0]
        chosen = scores[b, s][sel_mine[b, s]]
        kth = chosen.min()
        assert np.all(scores[b, s, diff] == kth), f"{what}: row ({b},{s}) differs beyond a tie: {diff}"
    return len(rows)


@pytest.mark.parametrize("name", list(spec.CONFIGS))
def test_nocache_matches_reference(name):
    c = spec.CONFIGS[name]
    params, x, pos = spec.make_params_and_inputs(c)
    g = c["seq"] // c["compress_ratio"]
    ref_sel = _sel(name, "nocache_sel", g)
    out, shared = M.layer_forward(params, _cfg(c), x, pos, select=ref_sel)
    _assert_close(_rows(name, out), FIX[f"{name}/nocache_out"], f"{name} output")
    assert np.array_equal(shared["index_k"], FIX[f"{name}/nocache_index_k"]), "published indexer keys"
    if f"{name}/nocache_compress_kv" in FIX:
        assert np.array_equal(shared["compress_kv"], FIX[f"{name}/nocache_compress_kv"]), "compressed latents"
    # the oracle's own selection: equal to the reference's up to ties
    _, own = M.layer_forward(params, _cfg(c), x, pos)
    n = _ties_only(ref_sel, own["selection"], own["scores"].numpy(), name)
    assert n <= max(2, c["seq"] * c["batch"] // 5), f"{n} rows decided by ties"


@pytest.mark.parametrize("name", list(spec.CONFIGS))
def test_chunked_cache_matches_reference(name):
    c = spec.CONFIGS[name]
    params, x, pos = spec.make_params_and_inputs(c)
    g = c["seq"] // c["compress_ratio"]
    ref_sel = _sel(name, "cached_sel", g)
    state = M.LayerState()
    outs, start = [], 0
    for n in spec.chunks(c):
        groups_now = (start + n) // c["compress_ratio"]
        o, _ = M.layer_forward(params, _cfg(c), x[:, start:start + n], pos[:, start:start + n], state,
                               select=ref_sel[:, start:start + n, :groups_now])
        outs.append(o)
        start += n
    out = np.concatenate(outs, 1)
    _assert_close(_rows(name, out), FIX[f"{name}/cached_out"], f"{name} chunked output")
    assert np.array_equal(state.index_k, FIX[f"{name}/cached_index_k"]), "indexer key cache"
    assert np.array_equal(state.window, FIX[f"{name}/cached_window"]), "window cache"
    assert state.entry_count == int(FIX[f"{name}/cached_entry_count"])
    if f"{name}/cached_compress_kv" in FIX:
        assert np.array_equal(state.compressed, FIX[f"{name}/cached_compress_kv"]), "compressed cache"
        _assert_close(state.buffer_kv, FIX[f"{name}/cached_buffer_kv"], "carried kv", rtol=1e-6)
        _assert_close(state.buffer_gate, FIX[f"{name}/cached_buffer_gate"], "carried gate", rtol=1e-6)


def test_selection_pins_the_mask_extension():
    """A plausible composition slip -- attending every compressed entry instead of the
    selected ones (the zero-padding the reference avoids, attention.py:202-214) -- moves the
    output far beyond the tolerance above."""
    c = spec.CONFIGS["small"]
    params, x, pos = spec.make_params_and_inputs(c)
    g = c["seq"] // c["compress_ratio"]
    every = np.ones((c["batch"], c["seq"], g), bool) & (np.arange(g) < (pos[..., None].numpy() + 1) // 4)
    out, _ = M.layer_forward(params, _cfg(c), x, pos, select=every)
    ref = FIX["small/nocache_out"]
    assert np.abs(out - ref).max() > 100 * 2e-5 * np.abs(ref).max()


# ---- multi-layer schedules ------------------------------------------------------------------

def _stack_cfg(c):
    return dict(c, rms_norm_eps=spec.RMS_NORM_EPS, compress_rope_theta=spec.COMPRESS_ROPE_THETA,
                rope_theta=spec.ROPE_THETA)


def _stack_groups(c, i):
    r = c["compress_ratios"][i]
    return c["seq"] // r if r else 0


def _index_layers(c):
    return [i for i in c["index_source_layer_ids"]]


def _candidates(name, c, run):
    """The reference's candidate mask (bool [B, S, G]) of a schedule with a candidate source."""
    if f"{name}/{run}_candidates" not in FIX:
        return None
    return _sel(name, f"{run}_candidates", _stack_groups(c, c["candidate_source_layer_id"]))


def _candidate_ties_only(ref, mine, scores, block, lens):
    """Candidate masks that differ only in blocks whose maxima tie with the weakest block
    kept (the reference's torch.topk orders equal block scores its own way); the block of
    the newest visible group is pinned in (indexer.py:33-35)."""
    b, s, g = ref.shape
    nb = -(-g // block)
    pad = np.full((b, s, nb * block), -np.inf, np.float32)
    pad[..., :g] = scores
    bmax = pad.reshape(b, s, nb, block).max(-1)
    np.put_along_axis(bmax, (lens[..., None] - 1) // block, np.inf, -1)
    for bi, si in np.argwhere((ref != mine).any(-1)):
        rb = ref[bi, si].reshape(-1)
        mb = mine[bi, si].reshape(-1)
        rblk = np.zeros(nb * block, bool)
        mblk = np.zeros(nb * block, bool)
        rblk[:g], mblk[:g] = rb, mb
        rblk = rblk.reshape(nb, block).any(-1)
        mblk = mblk.reshape(nb, block).any(-1)
        diff = np.nonzero(rblk != mblk)[0]
        kept = bmax[bi, si][mblk]
        weakest = kept[np.isfinite(kept)].min()
        assert np.all(bmax[bi, si, diff] == weakest), f"candidates of row ({bi},{si}) differ beyond a tie: {diff}"


@pytest.mark.parametrize("name", list(spec.STACKS))
def test_stack_nocache_matches_reference(name):
    """Every layer of the schedule (sliding-only, KV + index sources at ratios 1 / 2 / 4,
    Reuse, Reindex, candidate source and user, a left-padded batch) against the reference's
    modules run layer by layer with one shared dict, the reference's selections imposed."""
    c = spec.STACKS[name]
    params, xs, pos, live = spec.make_stack_params_and_inputs(c)
    sel = {i: _sel(name, f"nocache_sel{i}", _stack_groups(c, i)) for i in _index_layers(c)}
    cand = _candidates(name, c, "nocache")
    outs, pub = M.stack_forward(params, _stack_cfg(c), xs, pos, live=live, select=sel, candidates=cand)
    ref = FIX[f"{name}/nocache_out"]
    for i, o in enumerate(outs):
        _assert_close(o, ref[i], f"{name} layer {i} output")
    # the oracle's own candidate blocks: the reference's up to ties between equal block scores
    if cand is not None:
        _, own = M.stack_forward(params, _stack_cfg(c), xs, pos, live=live)
        src = c["candidate_source_layer_id"]
        lens = (pos.numpy() + 1) // c["compress_ratios"][src]
        _candidate_ties_only(cand, own[src]["candidates"], own[src]["scores"].numpy(), c["candidate_block_size"],
                             lens)
    # the oracle's own selections (on the reference's candidates): the reference's up to exact ties
    _, own = M.stack_forward(params, _stack_cfg(c), xs, pos, live=live, candidates=cand)
    for i in _index_layers(c):
        # (a ratio-1 group's early rows see few keys, many of them ReLU's exact zeros)
        n = _ties_only(sel[i], own[i]["selection"], own[i]["scores"].numpy(), f"{name} layer {i}")
        assert n <= c["seq"] * c["batch"] // 3, f"{name} layer {i}: {n} rows decided by ties"


@pytest.mark.parametrize("name", list(spec.STACKS))
def test_stack_chunked_cache_matches_reference(name):
    """The same schedules fed through per-layer caches (KV sources: DeepseekV41CSACache,
    the others: the sliding window) in two prefill chunks ending mid-group, then decode
    steps: outputs, windows, compressed caches, keys, group counts, the carried group."""
    c = spec.STACKS[name]
    params, xs, pos, live = spec.make_stack_params_and_inputs(c)
    layers = len(c["compress_ratios"])
    sel = {i: _sel(name, f"cached_sel{i}", _stack_groups(c, i)) for i in _index_layers(c)}
    cand = _candidates(name, c, "cached")
    states = [M.LayerState() for _ in range(layers)]
    outs, start = [], 0
    for n in spec.chunks(c):
        imposed = {i: s[:, start:start + n, :(start + n) // c["compress_ratios"][i]] for i, s in sel.items()}
        o, _ = M.stack_forward(params, _stack_cfg(c), [x[:, start:start + n] for x in xs], pos[:, start:start + n],
                               states, None if live is None else live[:, :start + n], imposed,
                               None if cand is None else cand[:, start:start + n])
        outs.append(np.stack(o))
        start += n
    out = np.concatenate(outs, 2)
    ref = FIX[f"{name}/cached_out"]
    for i in range(layers):
        _assert_close(out[i], ref[i], f"{name} layer {i} chunked output")
        assert np.array_equal(states[i].window, FIX[f"{name}/cached_window{i}"]), f"layer {i} window cache"
    for i in c["kv_source_layer_ids"]:
        st = states[i]
        assert st.entry_count == int(FIX[f"{name}/cached_entry_count{i}"]), f"layer {i} group count"
        assert np.array_equal(st.compressed, FIX[f"{name}/cached_compress_kv{i}"]), f"layer {i} compressed cache"
        if f"{name}/cached_index_k{i}" in FIX:
            assert np.array_equal(st.index_k, FIX[f"{name}/cached_index_k{i}"]), f"layer {i} key cache"
        if f"{name}/cached_buffer_kv{i}" in FIX:
            _assert_close(st.buffer_kv, FIX[f"{name}/cached_buffer_kv{i}"], f"layer {i} carried kv", rtol=1e-6)


def test_stack_pins_the_group_reset_and_the_padding():
    """Two composition slips the stack fixture catches: a second group appending to the
    first group's compressed entries (no reset at its KV source), and a padded batch whose
    pad tokens are attended."""
    c = spec.STACKS["two_groups"]
    params, xs, pos, _ = spec.make_stack_params_and_inputs(c)
    sel = {i: _sel("two_groups", f"nocache_sel{i}", _stack_groups(c, i)) for i in _index_layers(c)}
    keys = M._GROUP_KEYS
    ref = FIX["two_groups/nocache_out"][3]
    try:
        M._GROUP_KEYS = ()
        outs, _ = M.stack_forward(params, _stack_cfg(c), xs, pos, select=sel)
        assert np.abs(outs[3] - ref).max() > 100 * 2e-5 * np.abs(ref).max()
    finally:
        M._GROUP_KEYS = keys
    c = spec.STACKS["padded"]
    params, xs, pos, live = spec.make_stack_params_and_inputs(c)
    sel = {i: _sel("padded", f"nocache_sel{i}", _stack_groups(c, i)) for i in _index_layers(c)}
    outs, _ = M.stack_forward(params, _stack_cfg(c), xs, pos, live=None, select=sel)
    ref = FIX["padded/nocache_out"][0]
    assert np.abs(outs[0] - ref).max() > 100 * 2e-5 * np.abs(ref).max()
