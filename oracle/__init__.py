"""CPU restatement of unsloth-spectral's compressed-space decode path.

THIS PACKAGE IS TEST INFRASTRUCTURE, NOT THE PRODUCT.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only to check or time the reference
algorithm.  The shipped path (``unsloth_spectral`` + ``libspectral_hip.so``)
never imports anything from here and fails loudly when its HIP library is
missing.

Modules (each function cites the reference file:line it restates):

* ``oracle.quant``     -- INT8 symmetric quantisation
                          (unsloth_spectral/spectral_cache.py:452-516)
* ``oracle.rsvd``      -- batched randomized SVD
                          (unsloth_spectral/rsvd.py:74-157), plus the
                          float64 subspace-iteration variant that the HIP
                          kernel evaluates
* ``oracle.attention`` -- both decode paths with the reference's FP16 cast
                          points (unsloth_spectral/spectral_attention.py:117-349,
                          unsloth_spectral/kernels/spectral_attention.py:340-453,
                          544-601, 684-857) and the float64 closed form
* ``oracle.cache``     -- the tier manager (spectral_cache.py:164-319, 518-612)

How each part is pinned (see tests/test_oracle_*.py):

* quant     -- closed form, bit-exact: ties-to-even, all-zero input,
               absmax element -> +-127, sign symmetry, codes recovered from
               dequantised FP16 coefficients.
* rsvd      -- published known answer of the reference's seeded self-test
               (rsvd.py:160-220; err 0.022725, PHASE2_RSVD_OPTIMIZATION.md:40)
               reproduced from torch's seeded CPU generator; Q^T Q = I;
               Eckart-Young bound; exact SVD on inputs of rank <= k.
* attention -- float64 closed form (dense softmax attention over the
               dequantised keys rotated at the reference's angles), and the
               textbook HF rotate_half RoPE + eager attention for the
               absolute mode and for tail-only caches.
* cache     -- block counts / hot lengths / positions of the reference's
               own assertions (COLAB_LONG_CONTEXT_VALIDATION.py:255-275,
               test_gqa_fix.py:93-94) and get_kv round trips.
"""
