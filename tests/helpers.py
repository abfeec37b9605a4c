"""Shared test helpers."""
import numpy as np
import torch


def np_(t):
    if t is None:
        return None
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().numpy()
    return t


def assert_tuple_equal(got, ref, what=""):
    assert len(got) == len(ref) == 9, what
    for i, (g, r) in enumerate(zip(got, ref)):
        if r is None:
            assert g is None, f"{what} element {i}: expected None, got {type(g)}"
            continue
        if isinstance(r, (int, np.integer)):
            assert int(g) == int(r), f"{what} element {i}: {g} != {r}"
            continue
        g = np_(g)
        assert g.shape == r.shape, f"{what} element {i}: shape {g.shape} != {r.shape}"
        assert g.dtype == r.dtype, f"{what} element {i}: dtype {g.dtype} != {r.dtype}"
        if not np.array_equal(g, r):
            bad = np.argwhere(g != r)
            raise AssertionError(f"{what} element {i}: {len(bad)} mismatches, first at {bad[:5].tolist()} "
                                 f"got {g[tuple(bad[0])]} expected {r[tuple(bad[0])]}")


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / RMS(ref) -- the feature tolerance measure."""
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))) or 1.0
    return float(np.max(np.abs(got.astype(np.float64) - ref))) / rms


def sorted_keys(coords: np.ndarray, bits: int):
    from oracle import oracle as orc
    keys, _ = orc.flatten_sort(coords, bits == 64)
    return keys
