"""Parity oracle for the gsplat_amd HIP path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm (mc8max/gsplat 1.5.3) on the
host CPU:

* ``exact``     -- numpy + the C library built from ``exact_ref.c``: the integer
                   and bit-exact parts (projection validity/radii, tile sets,
                   sorted intersection ids, tile offsets, Adam, rasterizer
                   decision thresholds);
* ``torch_ref`` -- a float32/float64 PyTorch restatement of the differentiable
                   math (projection, SH, tile rasterizer, the full
                   ``rasterization()`` pipeline) whose backward comes from
                   autograd, independent of the hand-derived HIP backward.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU
baseline.  The product package ``gsplat_amd`` never imports it.
"""
