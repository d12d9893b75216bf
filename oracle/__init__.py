"""CPU oracle for the dense 3-D diffusion hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in float64 NumPy, what the reference
(MedMLX/lesiondiffusion-mlx v0.3.0) computes on its conditioned FP16 path:

* ``conv``      -- padding-1 3x3x3 / pointwise convolution, stride 1/2, nearest 2x
                   upsampling and its folded parity weights, packed weight layouts
                   (src/lesiondiffusion_mlx/_nax_conv.py, _spatial.py).
* ``norm``      -- GroupNorm statistics as a per-channel affine, GroupNorm, SiLU,
                   LayerNorm, erf-GELU (mlx_model.py:234-381).
* ``attention`` -- softmax(q k^T * scale + mask) v (tests/test_native_kernels.py:380-392,
                   mlx_model.py:443-493).
* ``unet``      -- the LDM 3-D UNet forward and the VQ decoder
                   (mlx_model.py:420-654, 720-819; _scaled_vq.py).
* ``sampling``  -- the uniform DDIM schedule and step (_schedules.py:11-39,
                   mlx_sampling.py:27-200).
* ``fixture_weights`` -- the seeded weight recipes behind the reference's recorded
                   Torch-CPU fixtures (tests/_fixture_models.py:31-157).
* ``vq``        -- the four-channel nearest-codebook search with its rounding points and
                   the straight-through quantize (_vq.py:12-82, mlx_model.py:742-803).
* ``torch_cpu`` -- the UNet and VQ decoder in torch fp32 on the CPU: ``bench.py``'s CPU
                   baseline for configs 3-5 (the same layer graphs as ``unet``).
* ``source_order`` -- the reference's Torch-CPU-ordered fp16 conv3d and Welford GroupNorm
                   cascade with every float32 rounding explicit (_source_half.py).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker. The product path (the HIP library
and its Python host layer) never imports it and has no CPU fallback.

Pinning: every function here is checked in ``tests/test_oracle.py`` against the
reference's recorded fixtures (copied under ``tests/golden/reference/``), against an
independent implementation (``torch`` CPU ops, brute-force loops on tiny inputs) or
against closed forms. Functions with no such check would be listed here as
"parity unpinned"; currently there are none.
"""
