"""CPU oracle for the Atlas memory-layer chunk scan.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the HIP library, the
``atlas_amd`` host package) imports, links or calls anything in this folder.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / the timed CPU baseline.

Contents
  atlas_ref.py     NumPy float64 restatement of the reference path
                   (rkstgr/atlas-jax, atlas_jax/memory_layer.py, kernels/,
                   model.py, optim.py), each function citing the lines it
                   follows, plus independent closed forms used to pin it
                   (SVD form of Polar-Express, per-token brute-force scan).
  cpu_baseline.py  torch-CPU float32 restatement of the reference's batched
                   non-fused JAX chunk loop; timed as the CPU baseline.

Parity status per function is listed in atlas_ref.py's header.
"""
