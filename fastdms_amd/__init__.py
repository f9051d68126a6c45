"""fastdms_amd — MI355X (gfx950) HIP implementation of FastDMS's compact-DMS
inference hot path.  The public engine API (``LLM``, ``SamplingParams``)
mirrors the reference's ``fastdms`` package; the kernels are in
``libfastdms_amd.so`` (C-ABI declared in include/fastdms_amd.h)."""
from .sampling_params import SamplingParams

__all__ = ["SamplingParams", "LLM"]


def __getattr__(name):
    if name == "LLM":
        from .llm import LLM
        return LLM
    raise AttributeError(name)
