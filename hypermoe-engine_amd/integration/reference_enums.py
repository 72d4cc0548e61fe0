#!/usr/bin/env python3
"""The three enumerator edits a maintainer makes to the reference so that it
knows HIP devices (src/tensor/Tensor.hpp:16-31, src/backend/Backend.hpp:15-18):

  tensor::DeviceType  gains HIP = 2, accepted by tensor::isValid and named
                      "HIP" by tensor::toString;
  backend::BackendKind gains Hip (value 2).

The adapter (HipMoEAdapter.hpp) uses exactly these values
(kHipDeviceType, kHipBackendKind).  Usage:

  python3 reference_enums.py REFERENCE_ROOT

edits REFERENCE_ROOT/src in place (run it on a checkout or a copy).  Each
edit is located by a short anchor and applied once; a missing anchor is an
error, and a tree that already has the edits is left as it is.
"""
from __future__ import annotations

import re
import sys
from pathlib import Path


def _edit(path: Path, done_re: str, edits: list[tuple[str, str]]) -> None:
    text = path.read_text()
    if re.search(done_re, text):
        return
    for pattern, repl in edits:
        new, n = re.subn(pattern, repl, text, count=1, flags=re.S)
        if n != 1:
            raise SystemExit(f"{path}: anchor not found: {pattern!r}")
        text = new
    path.write_text(text)


def apply(root: Path) -> None:
    src = root / "src"
    _edit(src / "tensor" / "Tensor.hpp", r"\bHIP\s*=\s*2\b", [
        # the enumerator, after CUDA
        (r"(enum class DeviceType[^{]*\{[^}]*?CUDA\s*=\s*1,)", r"\1\n    HIP = 2,"),
        # isValid accepts it
        (r"(return type == DeviceType::CPU \|\| type == DeviceType::CUDA)(;)",
         r"\1 || type == DeviceType::HIP\2"),
        # toString names it
        (r'(case DeviceType::CUDA: return "CUDA";)', r'\1\n    case DeviceType::HIP: return "HIP";'),
    ])
    _edit(src / "backend" / "Backend.hpp", r"enum class BackendKind\s*\{[^}]*\bHip\b", [
        (r"(enum class BackendKind\s*\{[^}]*?\bCuda,)", r"\1\n    Hip,"),
    ])


if __name__ == "__main__":
    if len(sys.argv) != 2:
        raise SystemExit("usage: reference_enums.py REFERENCE_ROOT")
    apply(Path(sys.argv[1]))
