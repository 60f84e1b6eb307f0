"""The MoE router's selection key (csrc/moe_route.h): one 64-bit key per (logit, expert), the
logit's bits mapped to an order-preserving unsigned in the high word (-0 taken as +0, NaN and
experts past E as key 0) and ~expert in the low word. Repeatedly taking the largest key must pick
the experts, in order, that repeated float argmax with ties to the lower index picks (the
reference's top-k, python/minisgl/layers/moe.py:1218-1227), including ties, signed zeros,
infinities, subnormals and NaN (never selected). This checks the mapping itself, restated in
numpy; the GPU route tests check the kernels' ids against the oracle bit for bit."""
import numpy as np
import pytest


def _key(v: np.float32, e: int) -> int:
    if np.isnan(v):
        return 0
    b = int(np.array(v, dtype=np.float32).view(np.uint32))
    if b == 0x80000000:
        b = 0
    u = (~b & 0xFFFFFFFF) if (b & 0x80000000) else (b | 0x80000000)
    return (u << 32) | (0xFFFFFFFF - e)


def _key_logit(k: int) -> np.float32:
    u = k >> 32
    b = (u & 0x7FFFFFFF) if (u & 0x80000000) else (~u & 0xFFFFFFFF)
    return np.array(b, dtype=np.uint32).view(np.float32)[()]


def _float_topk(v, k):
    used, out = set(), []
    for _ in range(k):
        bv, bi = -np.inf, 0x7FFFFFFF
        for e, x in enumerate(v):
            if e in used:
                continue
            if x > bv or (x == bv and e < bi):  # NaN compares false: never taken
                bv, bi = x, e
        if bi != 0x7FFFFFFF:
            used.add(bi)
        out.append((bv, bi))
    return out


def _key_topk(v, k):
    keys = [_key(x, e) for e, x in enumerate(v)]
    out = []
    for _ in range(k):
        top = max(keys)
        keys = [0 if x == top else x for x in keys]
        out.append((-np.inf, 0x7FFFFFFF) if top == 0 else (_key_logit(top), 0xFFFFFFFF - (top & 0xFFFFFFFF)))
    return out


_SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1e-40, -1e-40, 3.0, -3.0], np.float32)


@pytest.mark.parametrize("kind", ["normal", "ties", "specials"])
def test_key_order_matches_float_argmax(kind):
    rng = np.random.default_rng({"normal": 1, "ties": 2, "specials": 3}[kind])
    for _ in range(300):
        E = int(rng.integers(1, 300))
        k = int(rng.integers(1, min(E, 16) + 1))
        if kind == "specials":
            v = rng.choice(_SPECIALS, E)
        else:
            v = rng.standard_normal(E).astype(np.float32)
            if kind == "ties":
                v = (np.round(v * 2) / 2).astype(np.float32)
        for (a, i), (b, j) in zip(_float_topk(v, k), _key_topk(v, k)):
            assert i == j, (E, k, v)
            assert a == b or (np.isnan(a) and np.isnan(b)), (E, k, v)


def test_key_logit_round_trip():
    x = np.array([1.5, -2.25, np.inf, -np.inf, 0.0, 1e-40, -1e-40, 65504.0], np.float32)
    for e, v in enumerate(x):
        assert _key_logit(_key(v, e)) == v
    assert _key_logit(_key(np.float32(-0.0), 0)) == 0.0  # -0 is read back as +0
