"""CPU oracle for the TurboQuant KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

This package is a numpy restatement of the reference algorithm
(``mlx_lm/models/turboquant_cache.py`` in zayutaha/kaplumba).  It exists to
check the HIP product path and to time the CPU baseline.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker: nothing in ``kaplumba_amd/`` imports,
links or executes anything under ``oracle/``.

Pinning status of each function (how a plausible mistake would be caught):

* ``rht_signs``          -- pinned: numpy PCG64 stream, known-answer prefix.
* ``rotation_matrix``    -- pinned: orthogonality / det / sign-fixed diag(R)>0
                            invariants plus committed fixture.
* ``beta_codebook``      -- pinned: centroid condition against an independent
                            float64 quadrature of the Beta pdf, symmetry,
                            sqrt(d)-scaled closeness to the Gaussian table.
* ``gaussian_codebook``  -- pinned: published Lloyd-Max (Max 1960) levels.
* ``fwht_f32``/``rht_*`` -- pinned: float64 Sylvester-Hadamard closed form
                            (scipy.linalg.hadamard), involution, unit vectors.
* ``norm_f32``           -- pinned: float64 norm within 1 ulp, exact on
                            integer-valued inputs.
* ``quantize_rht``       -- pinned: brute-force nearest-centroid search,
                            strict ``>`` tie rule, zero vector special case.
* ``pack_lowbit``/``unpack_lowbit`` -- pinned: literal per-element loop of the
                            reference CPU branch, hand-computed words, round trip.
* ``attention``          -- pinned: float64 direct softmax, torch SDPA on the
                            dequantized cache, decode == last causal row.

The fp32 operation order of the quantizer (norm reduction tree, division,
Hadamard butterfly stage order, 1/sqrt(D) multiply, strict compare) is the
order the HIP append kernel implements; ``quantize_rht`` emulates it exactly
so packed bytes and norms can be compared bit for bit.  The reference's own
order inside MLX (``mx.linalg.norm``, ``mx.hadamard_transform``) cannot be
observed without MLX and is "parity unpinned" at the last ulp.
"""
