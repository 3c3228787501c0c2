"""Error metrics of the attention parity tests (imported by the test modules; not collected).

Two measures, both against a float64 evaluation of the oracle on the same (rounded) inputs:
- ``rel_err``: max |got - ref| / max |ref| over the whole tensor;
- ``row_rel_err``: the same per row (first dimension: a query or key/value node), each row
  against its own scale max |ref_row|, floored at ``floor`` x the tensor's scale, so a row whose
  reference is far below the tensor's maximum (the dK row of a rarely attended key) is held to its
  own size instead of to the largest row's.

The floor: bf16 results carry their own rounding (2^-9 of each value) and fp32 arithmetic
(~1e-7 of the terms), so 1e-3 leaves room under 2e-2. An fp32 row whose exact value cancels
(dq of a query with one edge is ~1e-6 of its terms: the softmax over one key is flat) keeps
fp32 rounding of those terms, ~1e-7 of the tensor's scale, so fp32 rows are floored at 0.1 —
still ten times stricter than the per-tensor bar for every row below a tenth of the maximum.
"""


def rel_err(got, ref) -> float:
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    scale = ref.abs().max().clamp_min(1e-30)
    return ((got - ref).abs().max() / scale).item()


def row_rel_err(got, ref, floor: float) -> float:
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    if ref.numel() == 0:
        return 0.0
    g = got.reshape(got.shape[0], -1)
    r = ref.reshape(ref.shape[0], -1)
    scale = r.abs().max().clamp_min(1e-30)
    row_scale = r.abs().amax(dim=1).clamp_min(floor * scale)
    return ((g - r).abs().amax(dim=1) / row_scale).max().item()


def default_floor(tol: float) -> float:
    return 1e-3 if tol >= 1e-3 else 0.1


def assert_close(name, got, ref, tol, floor=None) -> None:
    """Both measures within ``tol`` (the path's bar: 1e-5 fp32, 2e-2 bf16)."""
    floor = default_floor(tol) if floor is None else floor
    e = rel_err(got, ref)
    assert e < tol, f"{name}: tensor relative error {e:.3g} >= {tol}"
    er = row_rel_err(got, ref, floor)
    assert er < tol, f"{name}: per-row relative error {er:.3g} >= {tol} (row scale floored at {floor} x max)"
