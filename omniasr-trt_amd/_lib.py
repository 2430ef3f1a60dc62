"""Loader of ``libomniasr_mi355x.so``: the C ABI declared in ``include/omniasr_mi355x.h``.

The library is loaded with ``ctypes`` after ``torch``: both link ``libamdhip64.so.7``, so the loader
binds the library to the HIP runtime torch already loaded and torch's streams and device pointers
are valid in it.  A missing or unloadable library is an error, never a silent fallback.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must be loaded first: its HIP runtime is the one the library uses)

PATH = Path(__file__).resolve().with_name("libomniasr_mi355x.so")
ABI_VERSION = 3

OK = 0
F32, BF16 = 0, 1
ATTN_SEPARATE_COMBINE = 1
ATTN_SPLIT_K = 2
STATIC_WORKSPACE_BYTES = 32 << 20  # OMNI_STATIC_WORKSPACE_BYTES
STATIC_MAX_UNITS = 16384  # OMNI_STATIC_MAX_UNITS
SELECT_LOGP, SELECT_LOGITS = 0, 1  # OMNI_SELECT_*: what omni_beam_select's input rows hold

_P = c_void_p
_SIGNATURES = {
    "omni_status_string": (ctypes.c_char_p, [c_int]),
    "omni_abi_version": (c_int, []),
    "omni_rope_kv_append": (c_int, [_P, c_int64, _P, c_int64, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64,
                                    c_int64, c_int64, c_int64, c_int32, c_int32, c_int32, _P]),
    "omni_verify_attention_chunk": (c_int32, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "omni_verify_attention_workspace": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "omni_verify_attention": (c_int, [_P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, c_int32, c_int32, c_int32,
                                      c_int32, c_int32, c_int32, c_float, _P, _P, c_size_t, _P, c_int32, c_int32,
                                      _P]),
    "omni_verify_attention_static": (c_int, [_P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, c_int32, c_int32,
                                             c_int32, c_int32, c_int32, c_int32, c_float, _P, c_int32, c_int32, _P]),
    "omni_verify_attention_static_init": (c_int, []),
    "omni_beam_attention_workspace": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "omni_beam_attention": (c_int, [_P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, c_int64, c_int64,
                                    c_int64, c_int64, c_int64, _P, c_int64, _P, c_int32, c_int32, c_int32, c_int32,
                                    c_int32, c_int32, c_float, _P, _P, c_size_t, _P, c_int32, _P]),
    "omni_beam_gen_list": (c_int, [c_int32, c_int32, _P, c_int64, _P, c_int64, c_int64, c_int64, c_int64, _P, _P, _P,
                                   c_int64, _P]),
    "omni_beam_attention_listed": (c_int, [_P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, c_int64,
                                           c_int64, c_int64, c_int64, c_int64, _P, c_int64, _P, _P, _P, _P, c_int64,
                                           c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_float, _P, _P,
                                           c_size_t, _P, c_int32, _P]),
    "omni_prefill_attention": (c_int, [_P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, _P, c_int32, c_int32,
                                       c_int32, c_int32, c_float, _P, c_int32, _P]),
    "omni_propose": (c_int, [_P, c_int64, c_int64, _P, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, c_int32,
                             c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, _P, _P]),
    "omni_spec_prepare": (c_int, [_P, c_int64, c_int64, _P, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, c_int32,
                                  c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, _P, _P, _P,
                                  c_int64, _P, _P, _P, _P, _P]),
    "omni_accept": (c_int, [_P, _P, _P, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int32, c_int32, c_int64,
                            c_int64, _P]),
    "omni_greedy_accept": (c_int, [_P, c_int64, c_int32, c_int32, _P, _P, _P, c_int64, c_int64, _P, _P, _P, _P, _P,
                                   _P, c_int32, c_int32, c_int64, c_int64, _P]),
    "omni_beam_prepare": (c_int, [c_int32, c_int32, _P, _P, _P, _P, c_int64, c_int64, _P, _P, _P, _P, _P]),
    "omni_beam_select_workspace": (c_size_t, [c_int32, c_int32]),
    "omni_beam_select": (c_int, [_P, c_int64, c_int32, c_int32, c_int32, _P, _P, _P, c_int32, c_int64, _P, _P, _P,
                                 c_size_t, _P, c_int32, c_int32, _P]),
    "omni_rms_norm": (c_int, [_P, c_int64, _P, _P, c_int64, c_int32, c_int32, c_float, c_int32, _P]),
    "omni_silu_mul": (c_int, [_P, c_int64, _P, c_int64, c_int32, c_int32, c_int32, _P]),
    "omni_beam_take_over": (c_int, [c_int32, c_int32, c_int64, _P, _P, _P, c_int64, c_int64, _P, c_int64, c_int64,
                                    _P, _P, c_int32, _P, _P, _P, _P, _P, c_int64, c_int32, c_int32, _P]),
}

_lib: ctypes.CDLL | None = None


class KernelError(RuntimeError):
    """A launcher of the library returned an error status."""


def load() -> ctypes.CDLL:
    """The library, loaded once; raises if it is not built or does not match this package."""
    global _lib
    if _lib is None:
        if not PATH.exists():
            raise RuntimeError(f"{PATH} is not built: run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
        lib = ctypes.CDLL(str(PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.omni_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{PATH.name} has ABI version {version}, this package expects {ABI_VERSION}")
        _lib = lib
    return _lib


def symbols() -> list[str]:
    """The entry points this package binds (each declared in include/omniasr_mi355x.h)."""
    return sorted(_SIGNATURES)


def status_string(status: int) -> str:
    return load().omni_status_string(status).decode()


def check(status: int, what: str) -> None:
    if status != OK:
        raise KernelError(f"{what}: {status_string(status)} (status {status})")
