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


# 16-bit logits (bf16, fp16): one 32-bit key, the 16 bits mapped the same way in the high half and
# ~e in the low half (route_key16 in csrc/moe_route.h)
def _bits16(v: np.float32, dt: str) -> int:
    if dt == "fp16":
        return int(np.array(v, dtype=np.float16).view(np.uint16))
    return int(np.array(v, dtype=np.float32).view(np.uint32)) >> 16  # v is bf16-exact


def _val16(b: int, dt: str) -> np.float32:
    if dt == "fp16":
        return np.float32(np.array(b, dtype=np.uint16).view(np.float16))
    return np.array(b << 16, dtype=np.uint32).view(np.float32)[()]


def _key16(b: int, e: int, dt: str) -> int:
    if np.isnan(_val16(b, dt)):
        return 0
    b = 0 if b == 0x8000 else b
    u = (~b & 0xFFFF) if (b & 0x8000) else (b | 0x8000)
    return (u << 16) | (0xFFFF - e)


def _key16_topk(bits, k, dt):
    keys = [_key16(b, e, dt) for e, b in enumerate(bits)]
    out = []
    for _ in range(k):
        top = max(keys)
        keys = [0 if x == top else x for x in keys]
        if top == 0:
            out.append((-np.inf, 0x7FFFFFFF))
            continue
        u = top >> 16
        b = (u & 0x7FFF) if (u & 0x8000) else (~u & 0xFFFF)
        out.append((_val16(b, dt), 0xFFFF - (top & 0xFFFF)))
    return out


_SPECIALS16 = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 2.0 ** -133, -(2.0 ** -133), 2.0 ** -20, -(2.0 ** -20),
                        3.0, -3.0, 0.5], np.float32)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("kind", ["normal", "ties", "specials"])
def test_key16_order_matches_float_argmax(dt, kind):
    rng = np.random.default_rng({"normal": 4, "ties": 5, "specials": 6}[kind] + (dt == "fp16"))
    for _ in range(300):
        E = int(rng.integers(1, 300))
        k = int(rng.integers(1, min(E, 16) + 1))
        if kind == "specials":
            v = rng.choice(_SPECIALS16, E)
        else:
            v = rng.standard_normal(E).astype(np.float32)
            if kind == "ties":
                v = (np.round(v * 2) / 2).astype(np.float32)
        bits = [_bits16(x, dt) for x in v]
        vals = np.array([_val16(b, dt) for b in bits], np.float32)  # the logits as the kernel reads them
        for (a, i), (b, j) in zip(_float_topk(vals, k), _key16_topk(bits, k, dt)):
            assert i == j, (dt, E, k, vals)
            assert a == b or (np.isnan(a) and np.isnan(b)), (dt, E, k, vals)
