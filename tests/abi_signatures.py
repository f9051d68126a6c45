"""Parse exported C-ABI declarations (header or HIP sources) into ctypes
signature strings: 'p' pointer, 'i' int, 'l' int64_t, 'f' float."""
from __future__ import annotations

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _sig(args: str, name: str) -> str:
    out = ""
    for a in [x.strip() for x in args.replace("\n", " ").split(",") if x.strip()]:
        if a == "void":
            continue
        if "*" in a:
            out += "p"
        elif re.match(r"(const\s+)?int64_t\b", a):
            out += "l"
        elif re.match(r"(const\s+)?int\b", a):
            out += "i"
        elif re.match(r"(const\s+)?float\b", a):
            out += "f"
        else:
            raise ValueError(f"unhandled parameter {a!r} in {name}")
    return out


def header_signatures(path: Path | None = None) -> dict[str, str]:
    text = (path or ROOT / "include" / "fastdms_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return {m.group(1): _sig(m.group(2), m.group(1))
            for m in re.finditer(r"^int\s+(fdms_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M)}


def source_signatures() -> dict[str, str]:
    out = {}
    for f in sorted((ROOT / "fastdms_amd" / "csrc").glob("*.hip")):
        for m in re.finditer(r"FDMS_EXPORT\s+int\s+(\w+)\s*\(([^)]*)\)", f.read_text()):
            out[m.group(1)] = _sig(m.group(2), m.group(1))
    return out


if __name__ == "__main__":
    for k, v in source_signatures().items():
        print(f'    "{k}": "{v}",')
