"""CPU oracle for the sparse-attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference (pmonad/mzoo) computes on the
path the HIP library replaces.  It exists to check the product, never to be the
product: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  Nothing under ``mzoo_amd/`` imports it, and the product
path raises when the HIP library is missing instead of falling back to this code.

Modules
-------
``quant``      block FP8-e4m3 / FP4-e2m1 codecs (``owlet1/quant.py:1-86``) and the
               packed cache formats (656 B FP8-b128 latent entry, 132 B FP8 indexer
               key, 68 B MXFP4 indexer key).
``compressor`` the gated softmax pool + RMSNorm of ``owlet1/cache.py:142-172`` and
               ``owlet1/norm_rope.py:16-33`` with a pinned evaluation order, and the
               interleaved RoPE of ``owlet1/norm_rope.py:126-145``.
``attention``  ``golden`` / ``indexer_scores`` / ``topk_indices`` of
               ``layers/attn/golden_ref.py:57-243`` (torch fp32 on the CPU), the decode
               step built from them, and the lowest-index top-k tie rule.

Each function names the reference file:line it follows (paths relative to the
reference's repository root, ``src/mzoo/...``).
"""
