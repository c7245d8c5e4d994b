"""The product's seeded generators, pico_rand and pico_randn (libpico_amd.so).

pico_rand follows src/tensor.c:249-273: xorshift32 (shifts 13, 17, 5) on the
global x_state, each draw's top 23 bits as the mantissa of a float in [1, 2),
minus 1.  It must equal the oracle's restatement of that stream bit for bit
(the oracle's stream is itself pinned bit-exactly against the reference
compiled from its own sources, tests/test_oracle.py), and leave x_state where
n draws of the stream leave it.

pico_randn replaces src/tensor.c:348-367 with a flat Box-Muller over all numel
elements: pairs (u1, u2) of that stream with u1 = 1 - u in (0, 1], r =
sqrt(-2 ln u1), outputs r cos(2 pi u2) and r sin(2 pi u2), computed in double
and rounded once.  It is compared with a float64 numpy Box-Muller of the
oracle's stream (within 1e-6; libm and numpy may differ in the last bit of a
double) and with the oracle's fill (the same C expression: bit for bit), and
its moments are checked (mean 0, variance 1, no infinities from log(0)).
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from pico_amd.pico import Pico

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def P():
    return Pico()


def _state(P):
    return ctypes.c_uint32.in_dll(P.lib, "x_state")


def _xorshift(seed, n):
    s = seed
    out = np.empty(n, np.uint32)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = s
    return out, s


@pytest.mark.parametrize("shape", [[1], [7], [3, 5], [64, 784], [2, 3, 4, 5]])
def test_pico_rand_is_the_reference_stream(P, shape):
    seed = 20261201 + len(shape)
    n = int(np.prod(shape))
    st = _state(P)
    st.value = seed
    with P.arena(1 << 22):
        t = P.rand(P.lib.arena_ctx_current(), (ctypes.c_int64 * len(shape))(*shape), len(shape))
        assert P.shape(t) == tuple(shape)
        got = P.data(t)
    want = O.pico_rand(n, seed)
    assert got.dtype == np.float32 and np.array_equal(got, want)
    # the stream written out by hand: mantissa bits of the draw, minus one
    bits, last = _xorshift(seed, n)
    manual = ((bits >> 9) | np.uint32(0x3F800000)).view(np.float32) - np.float32(1.0)
    assert np.array_equal(got, manual)
    assert st.value == last  # x_state advanced by exactly n draws
    assert got.min() >= 0.0 and got.max() < 1.0


@pytest.mark.parametrize("n", [1, 2, 9, 1000, 200001])
def test_pico_randn_is_flat_box_muller(P, n):
    seed = 777 + n
    st = _state(P)
    st.value = seed
    with P.arena(1 << 24):
        t = P.randn(P.lib.arena_ctx_current(), (ctypes.c_int64 * 1)(n), 1)
        assert P.shape(t) == (n,)  # the requested shape, not a halved last dim
        got = P.data(t)
    m = (n + 1) // 2 * 2
    u = O.pico_rand(m, seed).astype(np.float64)
    u1, u2 = 1.0 - u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(m)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    want = z[:n].astype(np.float32)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got.astype(np.float64) - want)) <= 1e-6
    assert np.array_equal(got, O.normal(n, seed))
    _, last = _xorshift(seed, m)
    assert st.value == last  # ceil(n/2) pairs drawn
    if n >= 200000:
        assert abs(float(got.mean())) < 5e-3
        assert abs(float(got.var()) - 1.0) < 1e-2


def test_pico_randn_2d_shape(P):
    st = _state(P)
    st.value = 4242
    with P.arena(1 << 22):
        t = P.randn(P.lib.arena_ctx_current(), (ctypes.c_int64 * 2)(33, 17), 2)
        assert P.shape(t) == (33, 17)
        got = P.data(t)
    assert np.array_equal(got, O.normal(33 * 17, 4242))
