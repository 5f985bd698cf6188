"""CPU oracle for the dendritic tick -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

This package restates, on the CPU, the reference algorithm of NeuroSim-GPU's
dendritic matrix tick, PELS event tick, graph generator and weight quantizers.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker.  The shipped package
(``neurosim-gpu_amd/neurosim_gpu``) never imports it.

Pinning (each module's docstring names the checks that pin each function):

* ``topology``   -- random graph + coalescing CSR build (reference
  topology.py:8-115,213-247).  Pinned by the reference-held edge count of the
  brainwaves graph, by structural invariants and by a brute-force dictionary
  coalescer.  The reference's weight *bits* (topology_sha256) are platform
  dependent (torch's CPU normal sampler follows the host libm), so that SHA is
  not reproducible here; the trajectory pins below cover the weights to
  tolerance.
* ``dynamics``   -- the three-state update (reference compartmental.py:152-183,
  dynamics.py:41-61).  Pinned by closed forms (impulse decay, neutral
  parameters reduce to the point model exactly), by the reference-held FP64
  probe traces and by the reference-held brainwaves trajectory.
* ``runtime``    -- FP32 matrix tick and PELS tick (reference runtime.py:64-253,
  compartmental.py:274-348).  Pinned by a dense FP64 brute-force recurrence,
  the brainwaves trajectory and PELS invariants.
* ``precision``  -- fp8 e4m3 / NVFP4 encoders and decoders (reference
  precision.py:45-112).  Pinned exhaustively against torch's float8_e4m3fn
  conversion (a library routine implementing the OCP spec) and against a
  brute-force nearest-level search with ties to the even code.
"""
