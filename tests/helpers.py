"""Shared test helpers: geometry builders and tolerance checks."""
import torch

from fovi_amd.arch import knn_tables as T
from fovi_amd.sensing.coords import SamplingCoords


def layer_tables(res_in, res_out, k, side=None, fov=16, cmf_a=2.78):
    """Host tables of one log-polar layer: dict of coords, indices, slots, one-hot, CSR."""
    cin = SamplingCoords(fov, cmf_a, res_in, style="logpolar")
    cout = SamplingCoords(fov, cmf_a, res_out, style="logpolar")
    k = min(k, len(cin))
    idx, dist, src = T.knn_logpolar(cin.cortical, cout.cortical, k)
    ref, s = T.reference_grid(k, side_length=side)
    slots = T.local_rf_slots(idx, src, cin.cartesian, cout.cortical, cout.cartesian, ref)
    rf = T.slots_to_one_hot(slots, ref.shape[0])
    ptr, nbr = T.csr_tables(idx, slots, len(cin), ref.shape[0])
    return dict(cin=cin, cout=cout, k=k, idx=idx, dist=dist, slots=slots, rf=rf, ptr=ptr, nbr=nbr,
                V=ref.shape[0], side=s, n_in=len(cin), n_out=len(cout))


def rel_errs(got, ref):
    """(relative L2 error, max abs error / max |ref|)."""
    got = got.double().cpu()
    ref = ref.double().cpu()
    d = got - ref
    l2 = (d.norm() / ref.norm().clamp_min(1e-30)).item()
    mx = (d.abs().max() / ref.abs().max().clamp_min(1e-30)).item()
    return l2, mx


def assert_close_rel(got, ref, tol, what=""):
    l2, mx = rel_errs(got, ref)
    assert l2 <= tol and mx <= tol, f"{what}: rel L2 {l2:.3e}, rel max {mx:.3e} > {tol}"


def assert_mostly_bit_exact(got, ref, frac=0.999, what=""):
    """At least `frac` of the elements equal bit for bit (fp32 kernels that follow the
    oracle's rounding exactly; the remainder is covered by the tolerance check)."""
    eq = (got.cpu() == ref.cpu()).double().mean().item()
    assert eq >= frac, f"{what}: only {eq:.6f} of elements bit-exact"
