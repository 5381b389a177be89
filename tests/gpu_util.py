"""Shared helpers for the GPU parity tests."""
import numpy as np
import torch


def to_device(array: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).cuda()


def bits(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def assert_bitwise(got, expected, what: str = ""):
    g, e = bits(got), bits(expected)
    assert g.shape == e.shape, f"{what}: shape {g.shape} != {e.shape}"
    # NaN results compare as a class; every other value by its bits.
    gf, ef = g.view(np.float32), e.view(np.float32)
    same = (g == e) | (np.isnan(gf) & np.isnan(ef))
    if not same.all():
        where = np.argwhere(~same)[:5]
        samples = [(tuple(int(i) for i in w), float(gf[tuple(w)]), float(ef[tuple(w)])) for w in where]
        raise AssertionError(f"{what}: {int((~same).sum())} elements differ, e.g. {samples}")
