"""CPU oracle for the fovi hot path -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference's algorithm (nblauch/fovi, cited file:line in
each function) on the CPU with torch/numpy, used as the checker of the HIP
kernels. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it; the product package ``fovi_amd`` never
does, and has no CPU fallback.

Pinning (what checks each function beyond retyping its formula):
  * sampler_ref.transform_sampling_grid: closed-form fixation mapping
    (centre -> pixel centre, window edge -> window edge), exact fp32 values
    on power-of-two inputs.
  * sampler_ref.grid_sample_views: torch.nn.functional.grid_sample (library
    routine) and the textbook bilinear/nearest formulas on tiny images
    (sampler_ref.bilinear_numpy, brute force).
  * knnconv_ref.knnconv_forward: brute-force triple loop
    (knnconv_ref.knnconv_bruteforce) in float64, linearity, a one-hot
    weight that selects a single (slot, channel).
  * knnconv_ref.knnconv_fp8_forward / quantize_e4m3 (no reference
    counterpart): exhaustive nearest-value search over the e4m3 grid
    (e4m3_round_bruteforce), a closed form for constant inputs (slot sums =
    neighbour counts, rounded to e4m3 above 16), equality with
    knnconv_forward where every slot holds at most one neighbour.
  * knnpool_ref.knnpool_forward: the float64 loop form of the four modes
    (knnpool_ref.knnpool_bruteforce, NaN handled per definition), closed
    forms (max/avg/sum of a constant, of an arithmetic ramp), torch.nanmean /
    nansum on the same gathered tensor; knnpool_ref.gaussian_weights: a
    scalar loop of exp(-d^2 / 2 sigma^2) over min-max normalised distances,
    columns summing to 1 - 1e-8 relative, the largest weight at the nearest
    neighbour.
  * Gradients (torch autograd through knnconv_forward and knnpool_forward,
    in tests/test_knnconv_bwd.py and tests/test_knnpool.py): gradcheck
    (float64 finite differences), the closed form dW = dy^T a with the
    brute-force slot sums, the input gradient as the forward over the inverse
    neighbour table, and a float64 loop form of the pooling gradient rules
    (NaN features, pad tokens, the first maximum among ties).
  * policy_ref (the fixation draws): closed forms over one stream of
    uniforms (eval mode: only the centres, lo + (hi - lo) u; training: four
    draws per image, area, log-aspect, y, x), bit for bit; random_crop by
    invariants (the crop inside the image at integer corners, its area and
    aspect within the ranges up to rounding) and its clamped fallback.
  * The host tables the oracle consumes (sensor coordinates, kNN indices,
    ref slots; built by fovi_amd, not by this package) are pinned bit for bit
    by vectors the reference itself wrote (tests/golden/tables.npz, from
    tests/golden/make_golden.py), by closed forms (point counts, ring radii,
    lattice neighbourhoods) and by brute-force argsort on small grids.
"""
