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


def oracle_by_token_chunks(fn, hidden, *args, threads=None, chunk=None):
    """Runs an oracle block function (hm_oracle.moe_block / moe_block_limbs)
    over token chunks on host threads and concatenates (out, ids, scores).

    Exact, not approximate: routing, each expert row's MLP and the combine
    are per token in the reference (CpuRouterBackend::routeBatch routes token
    by token; every GEMM output row depends only on its own input row; the
    combine sums a token's own expert rows), so a chunk's rows come out with
    the same bits as in the whole batch.  ctypes releases the GIL for the C
    call, so the chunks run in parallel."""
    import os
    from concurrent.futures import ThreadPoolExecutor
    hidden = np.ascontiguousarray(hidden, np.float32)
    T = hidden.shape[0]
    if threads is None:
        threads = max(1, min(16, os.cpu_count() or 1))
    if chunk is None:
        chunk = max(1, -(-T // (4 * threads)))
    parts = [slice(i, min(T, i + chunk)) for i in range(0, T, chunk)]
    with ThreadPoolExecutor(threads) as ex:
        res = list(ex.map(lambda sl: fn(*args[:3], np.ascontiguousarray(hidden[sl]), *args[3:]),
                          parts))
    return tuple(np.concatenate([r[i] for r in res]) for i in range(3))


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
