"""The C ABI boundary without a GPU: the library loads, exports exactly what
include/moehip.h declares, the ctypes signatures cover it, and argument
checks fail loudly with a message (no kernel is launched by these calls)."""

import ctypes
import re
from pathlib import Path

import pytest

from distributedmoellm_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "moehip.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(moe_\w+)\s*\(", text, flags=re.M)))


def test_library_is_built_and_loads():
    assert _lib.LIB_PATH.exists(), "run python -m distributedmoellm_amd.build"
    assert _lib.load() is not None, _lib.why_not()


def test_every_declared_symbol_is_exported():
    names = header_functions()
    assert len(names) >= 14
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), f"{n} is declared in moehip.h but not exported"


def test_ctypes_signatures_match_header():
    assert set(header_functions()) == set(_lib.SIGNATURES)


def test_version_and_device_count_without_gpu():
    L = _lib.lib()
    assert L.moe_version() == 100
    assert L.moe_device_count() >= 0


def test_struct_layout():
    assert ctypes.sizeof(_lib.Q4Expert) == 40
    assert _lib.Q4Expert.xor8.offset == 32


@pytest.mark.parametrize("call,needle", [
    (lambda L: L.moe_q4_matmul_t(1, 1, 1, 1, 0, 8, 96, 7, 0, 1, None), "group size 7"),
    (lambda L: L.moe_q4_matmul_t(1, 1, 1, 1, 0, 8, 63, 63, 0, 1, None), "even"),
    (lambda L: L.moe_q4_matmul_t(None, 1, 1, 1, 0, 8, 64, 32, 0, 1, None), "null pointer"),
    (lambda L: L.moe_q8_matmul_t(1, -1, 1, 1, 0, 8, 64, 32, 1, None), "n=-1"),
    (lambda L: L.moe_gguf_matmul_t(1, 1, 1, 30, 8, 256, 1, None), "qtype 30"),
    (lambda L: L.moe_gguf_matmul_t(1, 1, 1, 12, 8, 100, 1, None), "multiple of 256"),
    (lambda L: L.moe_gguf_dequant(1, 8, 8, 33, 1, None), "multiple of 32"),
    (lambda L: L.moe_q4_layer(1, 64, 1, None, 1, 1, 1, 1, 4, 1, 1, 1, 1, 1, 64, 64, 32, 32, 1,
                              1, 10, None), "workspace"),
    (lambda L: L.moe_q4_layer_noalloc(1, 4096, 1, None, 1, 1, 1, 1, 2000, 1, 1, 1, 1, 1, 4096, 4096, 1536, 32, 1,
                                      None), "scratch"),
    (lambda L: L.moe_q4_layer_noalloc(1, 64, 1, None, 1, 1, 1, 1, 4, 1, 1, 1, 1, 1, 64, 64, 32, 24, 1,
                                      None), "group size 24"),
    (lambda L: L.moe_q4_layer(1, 64, 1, None, 1, 1, 1, 1, 4, 1, 1, 1, 1, 1, 64, 64, 32, 24, 1,
                              1, 10, None), "group size 24"),
    (lambda L: L.moe_combine(1, 8, 1, 1, 1, 1, 1, 0, 1, 8, 16, None), "ldy=8"),
    (lambda L: L.moe_combine(1, 16, 1, 1, 1, 1, 1, -1, 1, 16, 16, None), "max_pairs=-1"),
])
def test_bad_arguments_fail_with_a_message(call, needle):
    L = _lib.lib()
    rc = call(L)
    assert rc != 0
    assert needle in _lib.last_error()


def test_unsupported_is_its_own_code():
    """Formats and shapes the kernels do not take report MOE_EUNSUPPORTED, not MOE_EINVAL."""
    L = _lib.lib()
    assert L.moe_gguf_matmul_t(1, 1, 1, 30, 8, 256, 1, None) == _lib.MOE_EUNSUPPORTED    # BF16
    assert L.moe_gguf_dequant(1, 9, 8, 32, 1, None) == _lib.MOE_EUNSUPPORTED            # Q8_1
    assert L.moe_gguf_dequant(1, 1, 8, 32, 1, None) == _lib.MOE_EUNSUPPORTED            # F16
    # a prompt layer over more experts than a launch has grid rows, or with more
    # picks a token than the combine orders in LDS (nothing launched)
    args = (1, 128, 1, 4)
    assert L.moe_prefill_layer(*args, 70000, 8, 1, 1, 128, 128, 32, 1, 128, 1, 1 << 20, None) == \
        _lib.MOE_EUNSUPPORTED
    assert L.moe_prefill_layer(*args, 8192, 5000, 1, 1, 128, 128, 32, 1, 128, 1, 1 << 20, None) == \
        _lib.MOE_EUNSUPPORTED
    assert L.moe_prefill_layer(*args, 64, 65, 1, 1, 128, 128, 32, 1, 128, 1, 1 << 20, None) == _lib.MOE_EINVAL
    assert L.moe_route(1, 4, 64, 65, 1, 1, 1, None) == _lib.MOE_EINVAL     # k > E
    # every quantized type is taken; its rows must hold whole blocks
    for qt, per in ((2, 32), (3, 32), (6, 32), (7, 32), (10, 256), (11, 256), (13, 256), (14, 256)):
        assert L.moe_gguf_matmul_t(1, 1, 1, qt, 8, per + 16, 1, None) == _lib.MOE_EINVAL
        assert L.moe_gguf_dequant(1, qt, 8, per // 2, 1, None) == _lib.MOE_EINVAL
    assert L.moe_q4_grouped_ffn(1, 96, 1, 1, 1, 1, 4, 96, 128, 32, 1, 96, 1, 1 << 20, None) == _lib.MOE_EUNSUPPORTED
    assert "multiples of 128" in _lib.last_error()
    assert L.moe_q4_grouped_ffn(1, 128, 1, 1, 1, 1, 4, 128, 128, 16, 1, 128, 1, 1 << 20, None) == \
        _lib.MOE_EUNSUPPORTED
    assert L.moe_q4_grouped_ffn(1, 128, 1, 1, 1, 1, 4, -128, 128, 32, 1, 128, 1, 1 << 20, None) == _lib.MOE_EINVAL


def test_empty_calls_are_no_ops():
    L = _lib.lib()
    assert L.moe_q4_matmul_t(None, 0, None, None, 0, 8, 64, 32, 0, None, None) == 0
    assert L.moe_q4_layer(None, 64, None, None, 0, None, None, None, 0, None, None, None, 0, None, 64,
                          64, 32, 32, 0, None, 0, None) == 0
    # h and y, plus the activation limbs of the multi-row path (one 1 KB block
    # per 64 columns and pair, for the gate|up and the down inputs)
    assert L.moe_q4_layer_workspace(4, 2048, 768) >= 4 * (2 * 768 + 2048) * 4 + 4 * (2048 + 768) // 64 * 1024


def test_kernels_fail_loudly_without_gpu():
    from distributedmoellm_amd import kernels
    import numpy as np
    if kernels.ENABLED:
        pytest.skip("a GPU is present")
    assert kernels.WHY_DISABLED
    with pytest.raises(RuntimeError, match="not available"):
        kernels.q4_matmul_t(np.zeros((1, 64), np.float32), np.zeros((8, 32), np.uint8),
                            np.zeros((8, 2), np.float32), 32, False)


def test_int8_activation_calls_check_their_group_size():
    """The int8-activation layer call and the rounding take groups of 64 or
    multiples up to 512 (moelan/kernels.py:920-922); others are unsupported."""
    L = _lib.lib()
    assert L.moe_q4_layer_i8(1, 64, 1, None, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 64, 64, 64, 32, 1, 1, 1 << 20,
                             None) == _lib.MOE_EUNSUPPORTED
    assert "multiple of 64" in _lib.last_error()
    assert L.moe_q4_layer_i8(1, 192, 1, None, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 192, 192, 128, 128, 1, 1, 1 << 20,
                             None) == _lib.MOE_EUNSUPPORTED
    assert L.moe_round_q8(1, 96, None, 1, 96, 96, 1, 1, 1, None) == _lib.MOE_EUNSUPPORTED
    assert L.moe_round_q8(1, 1024, None, 1, 1024, 1024, 1, 1, 1, None) == _lib.MOE_EUNSUPPORTED
    assert L.moe_round_q8(1, 32, None, 1, 64, 64, 1, 1, 1, None) == _lib.MOE_EINVAL
    assert "ldx=32" in _lib.last_error()
    # too small a workspace is its own error, before anything runs
    assert L.moe_q4_layer_i8(1, 128, 1, None, 1, 1, 1, 1, 2, 1, 1, 1, 1, 1, 128, 128, 128, 64, 1, 256, 16,
                             None) == _lib.MOE_EWORKSPACE
    # nothing to do
    assert L.moe_q4_layer_i8(None, 128, None, None, 0, None, None, None, 0, None, None, None, 0, None, 128,
                             128, 128, 64, 0, None, 0, None) == 0
    assert L.moe_round_q8(None, 128, None, 0, 128, 64, None, None, None, None) == 0


def test_int8_activation_workspace():
    L = _lib.lib()

    def up(n):
        return (n + 255) // 256 * 256
    P, H, I, gs = 3, 2048, 768, 64
    # h, y, the rounded input rows with their d and s8, the rounded SiLU(gate)*up
    # rows with theirs, and the rounded row each pair reads
    want = (up(P * 2 * I * 4) + up(P * H * 4) + up(P * H) + 2 * up(P * (H // gs) * 4) + up(P * I)
            + 2 * up(P * (I // gs) * 4) + up(P * 4))
    assert L.moe_q4_layer_i8_workspace(P, H, I, gs) == want
    assert L.moe_q4_layer_i8_workspace(P, H, I, 96) == 0


def test_int8_act_for_follows_the_reference_rule(monkeypatch):
    """int8_act_for (moelan/kernels.py:920-922): on by default for groups of 64
    and multiples dividing H and I; MOELAN_INT8_ACT=0 turns it off."""
    from distributedmoellm_amd import kernels
    monkeypatch.setattr(kernels, "INT8_ACT", True)
    assert kernels.int8_act_for(2048, 768, 64)
    assert kernels.int8_act_for(2048, 768, 128)
    assert kernels.int8_act_for(1536, 384, 192)
    assert not kernels.int8_act_for(2048, 768, 32)
    assert not kernels.int8_act_for(2048, 800, 64)
    assert not kernels.int8_act_for(4096, 2048, 1024)
    monkeypatch.setattr(kernels, "INT8_ACT", False)
    assert not kernels.int8_act_for(2048, 768, 64)
