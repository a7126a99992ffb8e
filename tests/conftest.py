import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")

# Bar for the bf16 output against the reference (torch.allclose semantics).
ATOL = 1e-2
RTOL = 2e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU with ROCm")


def load_golden(name):
    path = os.path.join(GOLDEN_DIR, f"{name}.npz")
    if not os.path.exists(path):
        pytest.skip(f"golden fixture {name} not generated")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_lists(g):
    """Per-local-expert token lists from a golden fixture."""
    out, pos = [], 0
    for c in g["counts"].tolist():
        out.append(g["token_lists"][pos:pos + c].astype(np.int64))
        pos += c
    return out


def bf16_bits_to_f32(u16):
    u16 = np.asarray(u16, dtype=np.uint16)
    return (u16.astype(np.uint32) << 16).view(np.float32)


def assert_close_bf16(actual_f32, expected_f32, what=""):
    a = np.asarray(actual_f32, dtype=np.float64)
    e = np.asarray(expected_f32, dtype=np.float64)
    bad = np.abs(a - e) > ATOL + RTOL * np.abs(e)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements outside atol={ATOL} rtol={RTOL}; "
            f"first at {tuple(i)}: got {a[tuple(i)]!r} want {e[tuple(i)]!r}; "
            f"max abs err {np.abs(a - e).max():.4g}")
