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
