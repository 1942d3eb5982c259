"""CPU oracle for the TitanMAC sparse hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, what the reference computes on the path the
library accelerates, so the HIP kernels can be checked against it:

- ``oracle.masks``      attention masks (band and block-window), 64x64 tile
                        classification and the kernel work list;
- ``oracle.block_ell``  the Block-ELL index (splitmix64 sampler, validation,
                        transposition) and dense closed forms of the forward,
                        dX and dW-SDDMM products;
- ``oracle.attention``  masked softmax attention and the WindowedAttention
                        module forward.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU
baseline. The product path (``titans_core``) never imports it and has no CPU
fallback.

Pinning (what checks each function beyond its own formula; see the tests):
- masks.band_mask: closed-form pair count, per-row counts, brute-force
  predicate loops on small S, known totals (S=4096 -> 2,027,248 pairs).
- masks.blockwin_mask: literal re-execution of the reference's block loop on
  small S, cross-checked with the per-row interval form.
- masks.tile_kinds / schedule: brute-force tile reductions, known tile counts
  (S=4096, w=512, Np=16 -> 595 non-empty of 4096; 420 full, 175 partial).
- block_ell.SplitMix64: published splitmix64 output for seed 0.
- block_ell sampler / transpose: distinctness, sortedness, bijection checks,
  committed golden index arrays.
- block_ell products: brute-force block loops on tiny shapes, dense-GEMM
  special case (width = n_bcol), slot-permutation invariance, zero blocks.
- attention: torch's scaled_dot_product_attention (a library routine) with
  the same mask, single-key and constant-key closed forms.
"""
