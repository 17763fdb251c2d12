"""CPU oracle for the affine-quantized paged-attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``easymlx_amd`` imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and there only as the checker or the timed CPU
baseline -- never as the thing measured or shipped.

Contents (each function cites the reference file:line it restates):

* :mod:`oracle.affine` -- MLX 0.31.1 ``mx.quantize(..., mode="affine")`` /
  ``mx.dequantize`` for bits 4/8 (third-party algorithm, restated from MLX's
  public CPU kernel).  Bit-exactness against a real MLX install is
  **parity unpinned** (MLX is not importable here); the restatement is pinned
  by invariants (code range, exact edge/zero reconstruction, error bound,
  constant groups, packing order) and by a second, independent C restatement
  (``oracle/c/oracle.c``) that must agree bit for bit.
* :mod:`oracle.paged_attention` -- ``_paged_attention_reference``
  (``lib/python/easymlx/operations/kernels/unified_attention.py:187-281``)
  with the Metal kernels' edge semantics, the single-sequence causal path
  (``page_attention.py:84-133``) and the split-K merge (``page_attention.py:2006-2059``).
  Pinned by the reference tests' seeded cases (regenerated bit-exactly with
  numpy's PCG64), by ``torch.nn.functional.scaled_dot_product_attention`` on
  gathered dense K/V, and by closed-form special cases.
* :mod:`oracle.cache_write` -- the write-position arithmetic of
  ``PageCacheView.concatenate_to_cache`` (``caching/paged/cache.py:1088-1306``),
  pinned by the reference's ``rng(2)`` / ``rng(7)`` cache-write tests.
"""
