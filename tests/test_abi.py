"""The C ABI library loads, exports every symbol include/paged_infer_amd.h declares, and its
host-side entry points (no device needed) agree with the oracle: the quantizer is bit-exact
with the reference's quantize_rows_i8 restatement, block_hash with the FNV chain."""
import ctypes

import numpy as np
import pytest

import pia
from oracle import oracle as orc


def test_library_exports_every_declared_symbol():
    L = pia.lib()
    declared = pia.header_symbols()
    assert len(declared) > 40
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing
    assert set(declared) == set(pia._SIGS), set(declared) ^ set(pia._SIGS)
    assert pia.lib().pia_version().decode().startswith("paged-infer-amd")


def test_host_quantizer_bit_exact_with_oracle():
    rng = np.random.default_rng(11)
    cases = [rng.normal(0, 0.02, (37, 129)), rng.normal(0, 5, (8, 2048)), np.zeros((3, 7)),
             rng.integers(-300, 300, (16, 64)) / 4.0, np.array([[127, 63.5, -63.5, 0.5, -0.5, -0.0]]) / 128]
    for w in cases:
        w = w.astype(np.float32)
        q1, s1 = pia.quantize_rows_i8(w)
        q2, s2 = orc.quantize_rows_i8(w)
        assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


def test_synthetic_inputs_are_deterministic_and_normal():
    a = pia.synth_normal(42, 7, 100_001)
    b = pia.synth_normal(42, 7, 100_001)
    c = pia.synth_normal(42, 8, 100_001)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 5e-4 and abs(a.std() - 0.02) < 5e-4
    # Chunked generation equals one-shot (the threaded split does not change values).
    big = pia.synth_normal(3, 1, 3_000_001)
    assert np.array_equal(big[:1001], pia.synth_normal(3, 1, 1001))


def test_bf16_round_to_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.1415927, 1e-40, np.inf], np.float32)
    got = pia.f32_to_bf16(x)
    bits = x.view(np.uint32).astype(np.uint64)
    want = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(got, want)
    assert got[1] == 0x3F80  # halfway to even (down)
    assert got[2] == 0x3F82  # halfway to even (up)


def test_errors_are_status_codes_not_crashes():
    with pytest.raises(pia.PiaError, match="null"):
        pia.check(pia.lib().pia_kvm_create(4, 16, 1, None))
    h = ctypes.c_void_p()
    with pytest.raises(pia.PiaError, match="bad pool shape"):
        pia.check(pia.lib().pia_kvm_create(4, 0, 1, ctypes.byref(h)))
    # Kernel-tier entry points validate before touching the device.
    with pytest.raises(pia.PiaError, match="null"):
        pia.check(pia.lib().pia_qlinear_apply(None, None, None, None, None, 1, 1, 1))
    with pytest.raises(pia.PiaError, match="null context"):
        pia.check(pia.lib().pia_kv_write_dev(None, None, pia.KvLayout(1, 1, 1, 1, 4), None, None, None, None,
                                             1, 0, None))
    with pytest.raises(pia.PiaError, match="null context"):
        pia.check(pia.lib().pia_paged_attention_dev(None, None, None, None, pia.KvLayout(1, 1, 1, 1, 4), 1, None,
                                                    None, 1, 0, None))
