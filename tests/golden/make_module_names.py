"""Writes reference_module_names.json: the names each of the reference's
pybind11 kernel modules exports (its m.def / m.attr calls and the
ASDSL_DEF_PREQ_FP32 macro uses), read from the module sources as text.

Run in a container where the reference tree is mounted:
    python tests/golden/make_module_names.py [/root/reference]
The JSON is data for tests/test_kernels_api.py; nothing at test time reads the
reference tree.
"""

from __future__ import annotations

import json
import re
import sys
from pathlib import Path

MODULES = {
    "_native_gemv": "gemv_q4_avx2.cpp",
    "_native_gemv_q8": "gemv_q8_avx2.cpp",
    "_native_sparse_gemv": "gemv_sparse_avx2.cpp",
}

_PAT = re.compile(r'(?:\bm\.def|\bm\.attr|ASDSL_DEF_PREQ_FP32)\(\s*"([A-Za-z_0-9]+)"')


def module_names(src: str) -> list[str]:
    body = src[src.index("PYBIND11_MODULE("):]
    return sorted(set(_PAT.findall(body)))


def main(ref: Path) -> None:
    native = ref / "asdsl" / "kernels" / "native"
    out = {mod: module_names((native / fname).read_text(errors="replace")) for mod, fname in MODULES.items()}
    dst = Path(__file__).resolve().parent / "reference_module_names.json"
    dst.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(dst, {k: len(v) for k, v in out.items()})


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
