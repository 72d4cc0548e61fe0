"""Shared test setup.

CPU tests (no marker) check the oracle against the reference's known answers
and golden vectors, the host logic, and that the C ABI loads.  GPU tests
(@pytest.mark.gpu) are the parity tests proper: they call the HIP kernels
through the C ABI (include/hm_moe.h) and compare with the oracle.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO / "hypermoe-engine_amd"))
sys.path.insert(0, str(REPO / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def bits(a: np.ndarray) -> np.ndarray:
    """Bit pattern view for bit-exact float comparisons."""
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def assert_bitexact(actual, expected, what=""):
    actual, expected = np.asarray(actual), np.asarray(expected)
    assert actual.shape == expected.shape, (what, actual.shape, expected.shape)
    if actual.dtype.kind == "f":
        diff = bits(actual) != bits(expected)
    else:
        diff = actual != expected
    if diff.any():
        idx = np.argwhere(diff)[:5]
        pytest.fail(f"{what}: {int(diff.sum())} of {diff.size} elements differ; first at "
                    f"{idx.tolist()}: {actual[tuple(idx[0])]!r} vs {expected[tuple(idx[0])]!r}")


def assert_compare(actual, expected, atol, rtol, what=""):
    """CorrectnessOracle::compare semantics (src/validation/
    CorrectnessOracle.cpp:44-67): |a - b| <= atol + rtol*|b|, both finite."""
    a = np.asarray(actual, np.float64)
    b = np.asarray(expected, np.float64)
    ok = np.isfinite(a) & np.isfinite(b) & (np.abs(a - b) <= atol + rtol * np.abs(b))
    if not ok.all():
        i = np.argwhere(~ok)[0]
        pytest.fail(f"{what}: {int((~ok).sum())} mismatches (atol {atol}, rtol {rtol}); first "
                    f"{i.tolist()}: {a[tuple(i)]} vs {b[tuple(i)]}")


def normwise(actual, expected) -> float:
    a = np.asarray(actual, np.float64)
    b = np.asarray(expected, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


# ----------------------------------------------------------------- GPU ----
class Dev:
    """Device helpers over torch (device memory and the current stream only)."""

    def __init__(self):
        import torch
        self.torch = torch
        if not torch.cuda.is_available():
            pytest.skip("no GPU")
        from hmoe import capi
        self.capi = capi
        self.lib = capi.load()
        self.stream = torch.cuda.current_stream().cuda_stream
        # Device tensors created by to() stay alive until the test ends, so a
        # pointer taken inline (dev.to(x).data_ptr()) is never recycled by the
        # caching allocator for the next argument.
        self.keep = []

    def to(self, a: np.ndarray):
        t = self.torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
        self.keep.append(t)
        return t

    def empty(self, shape, dtype):
        tdt = {np.float32: self.torch.float32, np.int32: self.torch.int32,
               np.uint32: self.torch.int32, np.int8: self.torch.int8,
               np.float64: self.torch.float64, np.uint8: self.torch.uint8}[np.dtype(dtype).type]
        return self.torch.empty(shape, dtype=tdt, device="cuda")

    def zeros(self, shape, dtype):
        t = self.empty(shape, dtype)
        t.zero_()
        return t

    def host(self, t, dtype=None) -> np.ndarray:
        self.torch.cuda.synchronize()
        a = t.cpu().numpy()
        if dtype is not None:
            a = a.view(dtype)
        return a

    @staticmethod
    def p(t):
        return None if t is None else t.data_ptr()

    def call(self, name, *args):
        return self.capi.call(name, *args)

    def sync(self):
        self.torch.cuda.synchronize()


_DEV = None


@pytest.fixture
def dev():
    global _DEV
    if _DEV is None:
        print("[gpu] initialising device", flush=True)
        _DEV = Dev()
    yield _DEV
    _DEV.sync()
    _DEV.keep.clear()
