"""Parity helpers shared by the GPU tests.

Integer outputs (routing ids, counts, offsets, permutations) must be
bit-exact. bf16 outputs are checked two ways:

* stage-wise rounding exactness (:func:`assert_rounds_exactly`): each GPU
  stage is fed its own previous stage's output, and its bf16 result must be
  the nearest-even rounding of the float64-exact value of that stage; a
  neighbouring bf16 is admitted only where the exact value lies within
  d = 2^-15 |value| + 2^-20 sum|terms| of a rounding boundary (about 32 times
  the spread of an fp32 accumulation's rounding error). This is the
  element-wise bar: a wrong index, scale, sign or operand fails it grossly,
  and an extra rounding step anywhere in a stage fails it too.
* end to end against the full oracle (:func:`assert_block_output`): relative
  L2 error <= 2e-3, and every element inside the bounds of
  ``oracle.moe_output_interval`` -- the values the expert block can produce
  when each of its bf16 roundings (gate/up, act, down output, weighted
  product, slot sum, shared merge) takes any admissible value. A raw
  element-wise 1e-2 is not meaningful at these magnitudes (one bf16 step
  exceeds it above |x| = 2, and a one-step flip of an intermediate that two
  fp32 summation orders round differently propagates), so the bound is the
  propagated one; the max-abs error and the count beyond 1e-2 + one bf16 step
  of max(|ref|, mag) are reported beside it.
"""
import json
import os

import numpy as np
import torch

from oracle.qmoe_oracle import bf16_bits_to_f32, bf16_interval, compare

REL_L2 = 2e-3


def _steps(g, r):
    """Largest |g - r| in bf16 steps (one step = 2^(e-7) for a magnitude in
    [2^e, 2^(e+1))) of max(|r|, max|r| / 256), and max |r|. The floor keeps
    elements whose terms cancel to near zero from being measured in the
    steps of their own tiny value."""
    gv = bf16_bits_to_f32(g).astype(np.float64).ravel()
    rv = bf16_bits_to_f32(r).astype(np.float64).ravel()
    if rv.size == 0:
        return 0.0, 0.0
    a = np.maximum(np.abs(rv), max(np.abs(rv).max() / 256.0, 2.0 ** -126))
    step = np.exp2(np.floor(np.log2(a)) - 7)
    return float((np.abs(gv - rv) / step).max()), float(np.abs(rv).max())


def _record(kind, what, rel, mx, exact, beyond, outside=None, g=None, r=None):
    """Append one end-to-end parity figure to the file named by
    QMOE_PARITY_LOG (JSON lines), when set; tests/parity_summary.py turns
    the file into a table."""
    path = os.environ.get("QMOE_PARITY_LOG")
    if not path:
        return
    rec = {"kind": kind, "what": what, "rel_l2": rel, "max_abs": mx, "bitexact": exact, "beyond": beyond}
    if outside is not None:
        rec["outside_bounds"] = outside
    if g is not None:
        rec["max_steps"], rec["max_ref"] = _steps(g, r)
        rec["n"] = int(np.size(g))
    rec["test"] = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    with open(path, "a") as fh:
        fh.write(json.dumps(rec) + "\n")


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns on the host."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def to_dev(a: np.ndarray, device, dtype=None):
    """uint16 bf16 bits / int arrays -> device tensor."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)
    t = torch.from_numpy(a)
    return t.to(device) if dtype is None else t.to(device=device, dtype=dtype)


def _as_bits(got):
    return bits(got) if isinstance(got, torch.Tensor) else np.asarray(got).view(np.uint16)


def assert_bf16_close(got, ref_bits, what="", mag=None):
    g = _as_bits(got)
    r = np.asarray(ref_bits).view(np.uint16)
    rel, mx, beyond = compare(g, r.reshape(g.shape), None if mag is None else np.reshape(mag, g.shape))
    exact = float(np.mean(g == r.reshape(g.shape)))
    print(f"[parity] {what}: rel_l2={rel:.3e} max_abs={mx:.3e} bitexact={exact:.5f} beyond={beyond}", flush=True)
    _record("close", what, rel, mx, exact, beyond, g=g, r=r.reshape(g.shape))
    assert rel <= REL_L2, f"{what}: rel_l2 {rel:.3e} > {REL_L2}"
    assert beyond == 0, f"{what}: {beyond} elements beyond 1e-2 + one bf16 step of max(|ref|, mag)"
    return rel, mx, exact


def assert_block_output(got, ref_bits, bounds, what="", mag=None):
    """End-to-end check of an expert block's output: rel-L2 <= 2e-3 against the
    oracle and every element within ``bounds`` = (lo, hi) bf16 bits from
    ``oracle.moe_output_interval``."""
    g = _as_bits(got)
    r = np.asarray(ref_bits).view(np.uint16).reshape(g.shape)
    rel, mx, beyond = compare(g, r, None if mag is None else np.reshape(mag, g.shape))
    exact = float(np.mean(g == r))
    gv = bf16_bits_to_f32(g).astype(np.float64)
    lo = bf16_bits_to_f32(np.asarray(bounds[0]).view(np.uint16)).reshape(g.shape).astype(np.float64)
    hi = bf16_bits_to_f32(np.asarray(bounds[1]).view(np.uint16)).reshape(g.shape).astype(np.float64)
    out = np.flatnonzero(~((gv >= lo) & (gv <= hi)).ravel())
    print(f"[parity] {what}: rel_l2={rel:.3e} max_abs={mx:.3e} bitexact={exact:.5f} beyond={beyond} "
          f"outside_bounds={out.size}", flush=True)
    _record("block", what, rel, mx, exact, beyond, int(out.size), g=g, r=r)
    assert rel <= REL_L2, f"{what}: rel_l2 {rel:.3e} > {REL_L2}"
    if out.size:
        i = out[0]
        raise AssertionError(f"{what}: {out.size} of {g.size} elements outside their admissible bounds; first at "
                             f"{i}: got {gv.ravel()[i]} bounds [{lo.ravel()[i]}, {hi.ravel()[i]}]")
    return rel, mx, exact


def assert_equal_off_boundary(got, ref_bits, exact_f64, what=""):
    """got equals the oracle's bits wherever the float64 value it rounds lies
    clear of a bf16 rounding boundary (the two sides differ only in how their
    transcendental functions round in fp32); elsewhere it is one of the two
    admissible neighbours."""
    g = _as_bits(got).ravel()
    r = np.asarray(ref_bits).view(np.uint16).ravel()
    lo, hi = (b.ravel() for b in bf16_interval(np.asarray(exact_f64, dtype=np.float64)))
    differ = g != r
    on_boundary = lo != hi
    print(f"[parity] {what}: {int(differ.sum())} of {g.size} differ, all on a rounding boundary: "
          f"{bool(np.all(on_boundary[differ]))}", flush=True)
    bad = np.flatnonzero(differ & ~on_boundary)
    assert bad.size == 0, f"{what}: {bad.size} elements differ away from a rounding boundary (first {bad[0]})"
    bad = np.flatnonzero(differ & (g != lo) & (g != hi))
    assert bad.size == 0, f"{what}: {bad.size} elements outside their admissible roundings"


def assert_in_interval(got, lo_bits, hi_bits, what=""):
    """Every element of got lies in [lo, hi] (bf16 values, inclusive)."""
    g = bf16_bits_to_f32(_as_bits(got)).astype(np.float64)
    lo = bf16_bits_to_f32(np.asarray(lo_bits).view(np.uint16)).astype(np.float64)
    hi = bf16_bits_to_f32(np.asarray(hi_bits).view(np.uint16)).astype(np.float64)
    ok = (g >= lo) & (g <= hi)
    bad = np.flatnonzero(~ok.ravel())
    amb = float(np.mean(lo != hi))
    print(f"[stage] {what}: {g.size - bad.size}/{g.size} admissible (two-valued fraction {amb:.4f})", flush=True)
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {g.size} elements off their exact rounding; first at {i}: "
                             f"got {g.ravel()[i]} admissible [{lo.ravel()[i]}, {hi.ravel()[i]}]")


def assert_rounds_exactly(got, exact_f64, abs_sum=None, what=""):
    """GPU bf16 result == nearest-even rounding of the exact value (see module doc)."""
    assert_in_interval(got, *bf16_interval(exact_f64, abs_sum), what)


def assert_bf16_equal(got, ref_bits, what=""):
    g = _as_bits(got)
    r = np.asarray(ref_bits).view(np.uint16)
    bad = np.flatnonzero(g.ravel() != r.ravel())
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {r.size} elements differ; first at {i}: "
                             f"got {bf16_bits_to_f32(g.ravel()[i:i+1])[0]} ref {bf16_bits_to_f32(r.ravel()[i:i+1])[0]}")
