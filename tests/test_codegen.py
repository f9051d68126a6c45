"""Code-generation invariants of the HIP kernels, read from the compiler's
per-kernel resource report that the library build keeps beside each object
(fastdms_amd/_build/<source>.resources.txt).  No kernel may use scratch
memory or spill vector registers: a private array the compiler fails to keep
in registers goes through scratch memory, which costs HBM traffic and a wait
on every access (the expiry row mover once moved every row through scratch
that way, doubling its writes)."""
import re
from pathlib import Path

import pytest

PKG = Path(__file__).resolve().parents[1] / "fastdms_amd"


def test_no_kernel_uses_scratch_or_spills():
    sources = sorted((PKG / "csrc").glob("*.hip"))
    reports = [PKG / "_build" / (s.stem + ".resources.txt") for s in sources]
    if not all(r.exists() for r in reports):
        pytest.skip("library not built (run __graft_entry__.build())")
    bad, kernels = [], 0
    for src, rep in zip(sources, reports):
        for block in rep.read_text().split("Function Name: ")[1:]:
            name = block.split()[0]
            kernels += 1
            scratch = int(re.search(r"ScratchSize \[bytes/lane\]: (\d+)", block).group(1))
            spill = int(re.search(r"VGPRs Spill: (\d+)", block).group(1))
            if scratch or spill:
                bad.append(f"{src.name}: {name} scratch={scratch} spill={spill}")
    assert kernels > 100, "the resource reports list no kernels"
    assert not bad, "\n".join(bad)
