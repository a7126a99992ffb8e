import os
import sys

import numpy as np
import torch
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

from oracle import np_ref  # noqa: E402  (test infrastructure)


def quant_edge_rows():
    """bf16 rows whose blocks have closed-form quantisations: a power-of-two scale
    (amax 448 * 2^-3) with every e4m3 value and every midpoint between two (ties);
    an all-zero block; -0.0; bf16 subnormals; the largest bf16 values."""
    vals = np_ref.e4m3_table()
    fin = np.unique(vals[np.isfinite(vals) & (vals >= 0)])
    mids = (fin[:-1] + fin[1:]) / 2
    rows = np.zeros((3, 7168), dtype=np.float32)
    scale = 2.0 ** -3
    block = np.concatenate([[448.0], fin[:63], -mids[:64]])[:128] * scale  # exact in bf16
    rows[0, :128] = block
    rows[0, 128:256] = -block[::-1]
    rows[1, 256:384] = np.float32(2.0 ** -130) * np.arange(1, 129, dtype=np.float32)  # bf16 subnormals
    rows[1, 384] = -0.0
    rows[2, 512:640] = np.linspace(-3.3e38, 3.3e38, 128, dtype=np.float32)
    x = torch.from_numpy(rows).to(torch.bfloat16)
    assert torch.equal(x[0, :128].float(), torch.from_numpy(block.astype(np.float32)))
    return x
