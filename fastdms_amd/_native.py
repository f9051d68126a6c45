"""ctypes binding of libfastdms_amd.so (the C-ABI in include/fastdms_amd.h).

The product path has exactly one implementation: these HIP kernels.  If the
library is missing the first call raises; there is no CPU or Triton fallback.
Tensors cross the boundary as raw device pointers plus element strides, and
every launch goes on torch's current HIP stream, so the calls are capturable
in HIP graphs.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libfastdms_amd.so"

# dtype codes of the C-ABI
DT_F32, DT_F16, DT_BF16, DT_FP8 = 0, 1, 2, 3
_DTYPE_CODES = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}
if hasattr(torch, "float8_e4m3fn"):
    _DTYPE_CODES[torch.float8_e4m3fn] = DT_FP8

_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# name -> argument signature ('p' pointer, 'i' int32, 'l' int64, 'f' float)
SIGNATURES: dict[str, str] = {
    "fdms_abi_version": "",
    "fdms_copy_bytes": "pplip",
    "fdms_convert": "pipilp",
    "fdms_fp8_decode_hw": "pplp",
    "fdms_extract_dms_decisions": "pilllpllliiifffip",
    "fdms_streaming_pack_prepare": "pllpiiiiipllplllpppllllip",
    "fdms_streaming_pack_rank_scatter": "ppillllpllpiiiplllpllppilppplllllliiiiippp",
    "fdms_streaming_pack_scatter": "ppillllpllpllpllplppilpllplliiiiippp",
    "fdms_dms_rope_store_compact_decode": "pillppillllpllppilpllpllpiiiifffiiippp",
    "fdms_rope_inplace": "pillliipllpp",
    "fdms_store_compact_kvcache": "ppillllppilplliiippp",
    "fdms_compact_decode_attention": "pillppilpllpllipllpllppiiiiiifpllpppp",
    "fdms_fused_decode_attention": "pllpllpllpllppllpllfffipplpllpllpllppiiiiiifppppfp",
    "fdms_fused_decode_attention_noalloc": "pllpllpllpllppllpllfffipplpllpllplliiiiiifppppfp",
    "fdms_dms_expiry": "iplllplllplllplllppppllpiiiip",
    "fdms_prepare_decode_metadata": "plllplllpllliiip",
    "fdms_record_dms_decisions": "pllllpllllplllplllpipiiiip",
    "fdms_argmax_rows": "pillipp",
    "fdms_mfma_probe": "pppp",
    "fdms_prefill_attention": "pllpllpllpllpiiiiifp",
    "fdms_prefill_attention_varlen": "pllpllpllpllppiiiiifp",
    "fdms_rmsnorm": "pllippplplifpplip",
    "fdms_silu_mul": "pplip",
    "fdms_embedding_fp8": "plplplplip",
    "fdms_embedding_rmsnorm": "plpllpfplplip",
    "fdms_rmsnorm_partials": "pilppplplifpppplip",
    "fdms_quantize_fp8_rows": "pilliplpip",
    "fdms_linear_small_m": "pliipilppiipfplpliiippplpilppip",
    "fdms_linear_argmax_small_m": "pliipilppiiiipppppp",
    "fdms_linear_int4_small_m": "pliiplpilpiiipppppplp",
    "fdms_quantize_int4_groups": "pilliiiplplp",
    "fdms_fp8_rerank_topk": "pliiplpipipp",
    "fdms_paged_pack_prepare": "pllpiiiipllplllpppllllippppllpllipp",
    "fdms_paged_pack_scatter": "ppillllpllpiplllppilpppllllllplliiiiippp",
    "fdms_paged_prepare_decode": "plllplllplllplllplpipiiip",
    "fdms_paged_prepare_decode_plan": "plllplllplllplllplpipppliiiiiip",
    "fdms_paged_free": "piplllplllplllplpiip",
    "fdms_paged_expiry": "iplllplllplllplllplllplpppllpiiiip",
    "fdms_fused_decode_attention_paged": "pllpllpllpllppllpllfffipplpllipllpllppiiiiiifppppfp",
    "fdms_fused_decode_attention_planned": "pllpllpllpllpppllfffipplpllppiiiiifppppfp",
    "fdms_fp8_gemm": "plpplpppliiip",
}

_CT = {"p": _P, "i": _I, "l": _L, "f": _F}
_LIB: ctypes.CDLL | None = None


class NativeLibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it was not built."""
    global _LIB
    if _LIB is None:
        path = Path(os.environ.get("FASTDMS_AMD_LIB", LIB_PATH))
        if not path.exists():
            raise NativeLibraryMissing(
                f"fastdms_amd HIP library not found at {path}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`")
        handle = ctypes.CDLL(str(path))
        for name, sig in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = [_CT[c] for c in sig]
            fn.restype = ctypes.c_int
        _LIB = handle
    return _LIB


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed with HIP error {rc}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def require_cuda(*tensors: torch.Tensor, what: str = "fastdms_amd op") -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{what} requires tensors on the GPU (HIP device); got {t.device}")


def vec_width(head_dim: int, *tensors_and_offsets) -> int:
    """Largest element count (16/8/4/2/1) whose byte width keeps every given
    (tensor, element_strides...) access 16/8/4/2-byte aligned."""
    for v in (16, 8, 4, 2, 1):
        if head_dim % v:
            continue
        ok = True
        for t, strides in tensors_and_offsets:
            nbytes = v * t.element_size()
            if nbytes > 16:
                ok = False
                break
            if t.data_ptr() % nbytes:
                ok = False
                break
            if any((s * t.element_size()) % nbytes for s in strides):
                ok = False
                break
        if ok:
            return v
    return 1
