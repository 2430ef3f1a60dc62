"""The C ABI (CPU): the library loads and exports every entry point include/omniasr_mi355x.h declares, and the
argument checks that run before any launch answer with the documented status codes.  No kernel is launched."""

import ctypes
import re
from pathlib import Path

import pytest

from omniasr_trt_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "omniasr_mi355x.h"


def declared() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(omni_\w+)\s*\(", text))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = declared()
    assert {"omni_rope_kv_append", "omni_verify_attention", "omni_propose", "omni_accept",
            "omni_greedy_accept", "omni_spec_prepare"} <= names
    for name in names:
        assert hasattr(lib, name), name
    assert set(_lib.symbols()) == names  # the shim binds exactly what the header declares


def test_abi_version_and_status_text():
    lib = _lib.load()
    assert lib.omni_abi_version() == _lib.ABI_VERSION
    assert _lib.status_string(0) == "ok"
    for code in (-1, -2, -3, -4):
        assert _lib.status_string(code) not in ("ok", "unknown status")


def test_workspace_and_split_queries():
    lib = _lib.load()
    for rows, t, h, d, keys in ((8, 5, 32, 128, 2560), (8, 1, 8, 512, 2048), (1, 9, 32, 128, 1280), (4, 3, 2, 16, 256),
                                (1, 5, 2, 512, 256), (64, 3, 4, 256, 1024)):
        chunk = lib.omni_verify_attention_chunk(rows, t, h, d, keys)
        assert chunk % 32 == 0 and 32 <= chunk <= max(64, -(-keys // 32) * 32)
        splits = -(-keys // chunk)
        slots = max(splits, 2)  # split-K partials, or a unit's two halves
        units = rows * h * slots * t
        if d in (256, 512) and rows <= 64:  # the wide heads' balanced split-K: 256 workgroup slots over the heads
            units = max(units, h * max(rows, 256 // h) * t)
        want = -(-units * d * 4 // 256) * 256 + -(-units * 2 * 4 // 256) * 256
        assert lib.omni_verify_attention_workspace(rows, t, h, d, keys, 0) == want
    for groups, beams, h, d, keys in ((8, 5, 32, 128, 2560), (8, 5, 8, 512, 2304), (4, 16, 8, 256, 1024),
                                      (65, 2, 8, 512, 512)):
        chunk = lib.omni_verify_attention_chunk(groups, beams, h, d, keys)
        units = groups * h * max(-(-keys // chunk) + 1, 3) * beams  # key splits (or two halves) + generated keys
        if d in (256, 512) and groups <= 64:  # balanced: the heads' workgroup slots, one generated-keys slot per unit
            units = max(units, (h * max(groups, 256 // h) + groups * h) * beams)
        want = -(-units * d * 4 // 256) * 256 + -(-units * 2 * 4 // 256) * 256
        assert lib.omni_beam_attention_workspace(groups, beams, h, d, keys, 0) == want
    # config 3: 8 rows x 32 heads, keys 2560 -> 320 keys for 2048 waves, capped at 8 tiles per split
    assert lib.omni_verify_attention_chunk(8, 5, 32, 128, 2560) == 256
    # the real model's 8 heads x 512: whole-tile waves, 256 keys per split (measured fastest on MI355X)
    assert lib.omni_verify_attention_chunk(8, 5, 8, 512, 2048) == 256
    assert lib.omni_verify_attention_chunk(8, 5, 8, 512, 100) == 256  # one split covers every key


FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: every call below fails its checks before any launch


def test_argument_errors_before_launch():
    lib = _lib.load()
    # verify attention: 17 queries per row, an fp16 dtype, a too-small workspace
    args = [FAKE, FAKE, FAKE, 1 << 20, 1 << 16, 128, 4096, FAKE, 8, 17, 32, 128, 2560, 0, 0.1, FAKE, FAKE, 1 << 30,
            FAKE, 0, _lib.BF16, None]
    assert lib.omni_verify_attention(*args) == -3
    args[9] = 5
    args[-2] = 7
    assert lib.omni_verify_attention(*args) == -2
    args[-2] = _lib.BF16
    args[17] = 16
    assert lib.omni_verify_attention(*args) == -4
    args[17] = 1 << 30
    args[13] = 100  # a split that is not a multiple of 32 keys
    assert lib.omni_verify_attention(*args) == -1
    # rope: head_dim not a multiple of 8; nothing to do for zero tokens
    rope = [FAKE, 3 * 4 * 12, FAKE, 8192, FAKE, None, None, FAKE, FAKE, FAKE, 1, 1, 1, 8, 64, 5, 4, 12, _lib.BF16, None]
    assert lib.omni_rope_kv_append(*rope) == -3
    rope[15] = 0
    assert lib.omni_rope_kv_append(*rope) == 0
    # propose: k = 0 and a window wider than the kernel's
    reach = (ctypes.c_int32 * 8)(1, 1, 4, 2, 12, 4, 40, 6)
    prop = [FAKE, 2048, 2048, FAKE, 1024, 1024, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 8, 0, 8, 64, 160, 256, 256, 3,
            reach, None]
    assert lib.omni_propose(*prop) == -3
    prop[14] = 4
    prop[18] = 8192
    assert lib.omni_propose(*prop) == -3
    # accept: 65 tokens per row; greedy_accept: an int dtype for the logits
    acc = [FAKE, FAKE, FAKE, 2048, 2048, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 8, 65, 8188, 2, None]
    assert lib.omni_accept(*acc) == -3
    g = [FAKE, 10288, 10288, 5, FAKE, FAKE, FAKE, 2048, 2048, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 8, 5, 8188, 2, None]
    assert lib.omni_greedy_accept(*g) == -2


def test_workspaces_past_4_gib_are_refused_before_launch():
    """The partials are addressed with 32-bit offsets (16-byte buffer stores): a shape whose workspace reaches 4 GiB is
    refused with OMNI_ERR_SHAPE, before the workspace size or any pointer is looked at."""
    lib = _lib.load()
    rows, t, h, d, keys, chunk = 256, 16, 64, 128, 8192, 256
    assert lib.omni_verify_attention_workspace(rows, t, h, d, keys, chunk) >= 1 << 32
    args = [FAKE, FAKE, FAKE, 1 << 30, 1 << 20, 128, 8192, FAKE, rows, t, h, d, keys, chunk, 0.1, FAKE, FAKE, 1 << 40,
            FAKE, 0, _lib.BF16, None]
    assert lib.omni_verify_attention(*args) == -3
    args[8] = 8  # the same call at 8 rows fits: the missing workspace is what it then refuses
    args[17] = 16
    assert lib.omni_verify_attention(*args) == -4
    groups, beams, h, d, keys = 64, 16, 64, 512, 8192
    assert lib.omni_beam_attention_workspace(groups, beams, h, d, keys, 32) >= 1 << 32
    beam = [FAKE, FAKE, FAKE, 1 << 30, 1 << 24, 512, 8192, FAKE, FAKE, FAKE, 1 << 30, 1 << 24, 512, 64, 1024, FAKE, 64,
            FAKE, groups, beams, h, d, keys, 32, 0.1, FAKE, FAKE, 1 << 40, FAKE, _lib.BF16, None]
    assert lib.omni_beam_attention(*beam) == -3
    beam[18], beam[27] = 2, 16  # 2 groups fit: the missing workspace is what it then refuses
    assert lib.omni_beam_attention(*beam) == -4


def test_kernels_refuse_without_gpu():
    import torch

    from omniasr_trt_amd import kernels

    assert kernels.available(torch.device("cpu")) is False
    with pytest.raises(Exception):
        kernels.rope_kv(torch.zeros(1, 48), torch.zeros(8, 4, 2), torch.zeros(1, dtype=torch.long),
                        torch.zeros(1, 4, 8, 8), torch.zeros(1, 4, 8, 8), 2)


def test_static_scratch_refuses_oversized_shapes_before_launch():
    """omni_verify_attention_static: a shape whose workspace exceeds the static scratch, or with more (row, head)
    units than it has tickets, is refused with OMNI_ERR_WORKSPACE before anything is looked up or launched."""
    lib = _lib.load()
    assert lib.omni_verify_attention_workspace(8, 16, 32, 128, 8192, 64) > _lib.STATIC_WORKSPACE_BYTES
    args = [FAKE, FAKE, FAKE, 1 << 20, 1 << 16, 128, 8192, FAKE, 8, 16, 32, 128, 8192, 64, 0.1, FAKE, 0, _lib.BF16,
            None]
    assert lib.omni_verify_attention_static(*args) == -4
    args[8], args[9], args[10], args[11], args[12], args[13] = 1024, 1, 32, 16, 256, 256  # 32768 units > 16384
    assert lib.omni_verify_attention_workspace(1024, 1, 32, 16, 256, 256) < _lib.STATIC_WORKSPACE_BYTES
    assert lib.omni_verify_attention_static(*args) == -4
    args[9] = 17  # the shape checks of omni_verify_attention come first
    assert lib.omni_verify_attention_static(*args) == -3


def test_layer_op_argument_errors_before_launch():
    lib = _lib.load()
    assert lib.omni_rms_norm(FAKE, 4096, FAKE, FAKE, 4096, 40, 4096, 1e-5, _lib.F32, None) == -2
    assert lib.omni_rms_norm(FAKE, 4096, FAKE, FAKE, 4096, 40, 4100, 1e-5, _lib.BF16, None) == -3  # not 8 | dim
    assert lib.omni_rms_norm(FAKE, 16384, FAKE, FAKE, 16384, 40, 16384, 1e-5, _lib.BF16, None) == -3  # > 8192
    assert lib.omni_rms_norm(FAKE, 4000, FAKE, FAKE, 4096, 40, 4096, 1e-5, _lib.BF16, None) == -1  # stride < dim
    assert lib.omni_rms_norm(None, 4096, None, None, 4096, 0, 4096, 1e-5, _lib.BF16, None) == 0  # nothing to do
    assert lib.omni_silu_mul(FAKE, 22016, FAKE, 11008, 40, 11008, _lib.F32, None) == -2
    assert lib.omni_silu_mul(FAKE, 22020, FAKE, 11010, 40, 11010, _lib.BF16, None) == -3
    assert lib.omni_silu_mul(FAKE, 11008, FAKE, 11008, 40, 11008, _lib.BF16, None) == -1  # stride < 2 * ffn
