"""CPU checks of the C-ABI library: it loads, exports every symbol the
header declares, and its host-only encoders match the reference converter's
golden vectors. No GPU compute is issued here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import prana_amd as P
from prana_amd import _lib
from tests import fixtures as fx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden", "kquant_encoder_vectors.npz")


def header_functions():
    text = open(os.path.join(ROOT, "include", "prana_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(prana_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(_lib.LIB_PATH)
    names = header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(header_functions()) == set(_lib.exported_symbols())


def test_error_reporting_without_gpu_work():
    lib = _lib.load()
    assert isinstance(lib.prana_last_error(), bytes)
    # an invalid encoder call fails with a message and no abort
    syn = _lib.load_synth()
    rc = syn.prana_quantize_tensor(P.Q4_K, None, 1, 100, None, 0)
    assert rc == -1
    assert b"null" in syn.prana_synth_last_error()


def test_product_library_carries_no_fixture_encoders():
    lib = C.CDLL(_lib.LIB_PATH)
    for name in ("prana_quantize_tensor", "prana_synth_normal", "prana_synth_tensor"):
        assert not hasattr(lib, name), name
    syn = C.CDLL(_lib.SYNTH_PATH)
    for name in _lib._SYNTH_SIGS:
        assert hasattr(syn, name), name


def test_ggml_nbytes():
    assert P.ggml_nbytes(P.Q4_0, 64) == 36
    assert P.ggml_nbytes(P.Q8_0, 64) == 68
    assert P.ggml_nbytes(P.Q4_K, 512) == 288
    assert P.ggml_nbytes(P.Q6_K, 512) == 420
    assert P.ggml_nbytes(P.Q4_0, 33) == 0


@pytest.mark.parametrize("key,ty", [("q4k", P.Q4_K), ("q6k", P.Q6_K)])
def test_kquant_encoders_match_reference_converter(key, ty):
    g = np.load(GOLD)
    x = g["inputs"].astype(np.float32)
    got = P.quantize_tensor(ty, x).reshape(x.shape[0], -1)
    assert np.array_equal(got, g[key])


def test_q8_0_encoder_properties():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    raw = P.quantize_tensor(P.Q8_0, x)
    deq = fx.np_dequant(fx.Q8_0, raw, 4, 128)
    d = raw.reshape(-1, 34)[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    # d = f16(amax/127); every element within half a quantization step
    amax = np.abs(x.reshape(-1, 32)).max(1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    # q is rounded against the f32 d while the stored d is f16: the bound is
    # half a step plus 127 times the f16 rounding of d.
    step = np.repeat(amax / 127, 32).reshape(4, 128)
    d16err = np.repeat(np.abs(d - amax / 127), 32).reshape(4, 128)
    assert np.all(np.abs(deq - x) <= 0.5 * step * 1.001 + 127 * d16err)


def test_q4_0_encoder_properties():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    raw = P.quantize_tensor(P.Q4_0, x).reshape(-1, 18)
    deq = fx.np_dequant(fx.Q4_0, raw, 4, 128).reshape(-1, 32)
    xb = x.reshape(-1, 32)
    for b in range(xb.shape[0]):
        i = np.abs(xb[b]).argmax()
        d = raw[b, 0:2].copy().view(np.float16).astype(np.float32)[0]
        assert d == np.float16(xb[b, i] / np.float32(-8.0)).astype(np.float32)
        # the extreme element maps to nibble 0 (value -8*d = max)
        assert (raw[b, 2 + i % 16] >> (4 * (i // 16))) & 0xF == 0
        # half a step inside (-8d, 7d]; the clamped end (nibble 16 -> 15) is
        # one full step off
        err = np.abs(deq[b] - xb[b])
        assert np.all(err <= abs(d) * 1.01)
        inner = np.abs(xb[b]) < abs(d) * 7
        assert np.all(err[inner] <= abs(d) * 0.5 * 1.01)


def test_synth_is_deterministic_and_normal():
    a = P.synth_normal(123, 0.02, 1 << 18)
    b = P.synth_normal(123, 0.02, 1 << 18)
    c = P.synth_normal(124, 0.02, 1 << 18)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    t1 = P.synth_tensor(P.Q4_0, 64, 4096, 9, 0.02)
    t2 = P.quantize_tensor(P.Q4_0, P.synth_normal(9, 0.02, 64 * 4096).reshape(64, 4096))
    assert np.array_equal(t1, t2)
