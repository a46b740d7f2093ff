"""CPU oracle for the fovi hot path -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference's algorithm (nblauch/fovi, cited file:line in
each function) on the CPU with torch/numpy, used as the checker of the HIP
kernels. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it; the product package ``fovi_amd`` never
does, and has no CPU fallback.

Pinning (what checks each function beyond retyping its formula):
  * sampler_ref.transform_sampling_grid: closed-form fixation mapping
    (centre -> pixel centre, window edge -> window edge), exact fp32 values
    on power-of-two inputs; golden fixtures from the reference.
  * sampler_ref.grid_sample_views: torch.nn.functional.grid_sample (library
    routine) and the textbook bilinear/nearest formulas on tiny images
    (sampler_ref.bilinear_numpy, brute force).
  * knnconv_ref.knnconv_forward: brute-force triple loop
    (knnconv_ref.knnconv_bruteforce) in float64, linearity, a one-hot
    weight that selects a single (slot, channel); golden fixtures.
  * geometry_ref: closed forms (point counts, ring radii, lattice
    neighbourhoods) and golden fixtures written by the reference itself
    (tests/golden/make_golden.py).
"""
