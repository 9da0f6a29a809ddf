"""Writes tests/golden/known_answers.npz: known-answer cases for the record format and decode whose
expected values follow from how the inputs are built, not from running a quantizer.

    python tests/golden/make_known_answers.py

Format being pinned (reference: kushkash/kush/quant.mojo:25-87, kushkash/_ops.py:29-31): per page and
kv head a record [kq 32*DC | vq 32*DC | ks D fp16 | kb D fp16 | vs 32 fp16 | vb 32 fp16], DC = D (int8)
or D/2 (int4, byte j = code[j] & 0xF | code[j + D/2] << 4); K is quantized per channel over the
page's 32 tokens, V per token over its D dims; s = fp16((max - min) / (2^bits - 1)),
b = fp16(min + s * 2^(bits-1)), code = clamp(round((x - b) / s), -2^(bits-1), 2^(bits-1) - 1).

Cases (all inputs fp32, seed 0):
  exact_D{64,128}_b{4,8}: one sequence of 64 tokens (two full pages), 2 kv heads, 3 q heads per kv
    head. Every K channel of a page and every V row is b + c * s with s a dyadic number exact in fp16,
    b a dyadic multiple of s exact in fp16, and integer codes c in range that reach both extremes.
    Then max - min = (2^bits - 1) s exactly, so the quantizer must return exactly s, b and c; the
    expected record bytes are packed from them. Decode: K and V dequantize exactly, so the expected
    attention output is float64 softmax(q K^T scale) V over the original K, V (q random, and q = 0:
    the mean of V).
  ties_D64_b4: s = 1, b = 0, extremes -8 and 7 in every channel / row, the other values c + 1/2:
    codes round half to even (the rule of torch.round, which the reference's own test restatement
    uses, tests/test_cpu.py:16-24).
  const_D64_b{4,8}: one constant K channel (0.1) and one constant V row (-0.3): s = 0, code 0 and
    b = fp16(value).
  clamp_D64_b4: a K channel with values k 2^-24 (k = 0..16) and 16.5 2^-24: (max - min) / 15 is
    1.1 2^-24, which fp16 rounds to the subnormal 2^-24, so b = 8 2^-24 and x = 16 2^-24 and
    16.5 2^-24 land at 8 and 8.5 levels: both clamp to 7.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

PAGE = 32
OUT = Path(__file__).resolve().parent / "known_answers.npz"


def dc(D: int, bits: int) -> int:
    return D if bits == 8 else D // 2


def pack_codes(c: np.ndarray, D: int, bits: int) -> np.ndarray:
    c = c.astype(np.int64)
    if bits == 8:
        return (c & 0xFF).astype(np.uint8)
    return ((c[..., :D // 2] & 0xF) | ((c[..., D // 2:] & 0xF) << 4)).astype(np.uint8)


def f16_bytes(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x.astype("<f2")).view(np.uint8).ravel()


def record(kc, ks, kb, vc, vs, vb, D, bits) -> np.ndarray:
    """kc, vc [32, D] integer codes; ks, kb [D]; vs, vb [32] (fp16-exact values)."""
    return np.concatenate([pack_codes(kc, D, bits).ravel(), pack_codes(vc, D, bits).ravel(),
                           f16_bytes(ks), f16_bytes(kb), f16_bytes(vs), f16_bytes(vb)])


def exact_f16(x: np.ndarray) -> None:
    assert np.array_equal(x.astype(np.float16).astype(np.float64), x), "value not exact in fp16"


def dyadic_params(rng, n: int, bits: int):
    """n (scale, offset) pairs: scale 2^e * m (m in {1, 1.25, 1.5, 1.75}), offset = scale * k / 4."""
    e = rng.integers(-5, 2, n)
    m = rng.choice([1.0, 1.25, 1.5, 1.75], n)
    s = np.ldexp(m, e)
    b = s * rng.integers(-64, 65, n) / 4.0
    exact_f16(s)
    exact_f16(b)
    return s, b


def codes_with_extremes(rng, shape, axis: int, bits: int) -> np.ndarray:
    """Random codes in [-H, H-1] whose every line along `axis` holds both -H and H-1."""
    H = 2 ** (bits - 1)
    c = rng.integers(-H, H, shape)
    idx = [slice(None)] * len(shape)
    idx[axis] = 0
    c[tuple(idx)] = -H
    idx[axis] = 1
    c[tuple(idx)] = H - 1
    return c


def exact_case(rng, D: int, bits: int, Hkv: int = 2, G: int = 3, pages: int = 2):
    n = pages * PAGE
    K = np.zeros((Hkv, n, D))
    V = np.zeros((Hkv, n, D))
    recs = np.zeros((pages, Hkv, 64 * dc(D, bits) + 4 * D + 128), np.uint8)
    for p in range(pages):
        for h in range(Hkv):
            ks, kb = dyadic_params(rng, D, bits)
            kc = codes_with_extremes(rng, (PAGE, D), 0, bits)      # per channel over tokens
            vs, vb = dyadic_params(rng, PAGE, bits)
            vc = codes_with_extremes(rng, (PAGE, D), 1, bits)      # per token over dims
            K[h, p * PAGE:(p + 1) * PAGE] = kb[None, :] + kc * ks[None, :]
            V[h, p * PAGE:(p + 1) * PAGE] = vb[:, None] + vc * vs[:, None]
            recs[p, h] = record(kc, ks, kb, vc, vs, vb, D, bits)
    assert np.array_equal(K.astype(np.float32).astype(np.float64), K)
    assert np.array_equal(V.astype(np.float32).astype(np.float64), V)
    q = rng.standard_normal((Hkv * G, D)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)

    def attend(qq):
        out = np.zeros((Hkv * G, D))
        for hq in range(Hkv * G):
            h = hq // G
            sc = (K[h] @ qq[hq].astype(np.float64)) * np.float64(np.float32(scale))
            w = np.exp(sc - sc.max())
            out[hq] = (w / w.sum()) @ V[h]
        return out
    return dict(K=K.astype(np.float32), V=V.astype(np.float32), rec=recs, q=q, scale=np.float32(scale),
                out=attend(q), out_q0=attend(np.zeros_like(q)), G=np.int64(G))


def ties_case():
    D, bits = 64, 4
    K = np.zeros((PAGE, D))
    V = np.zeros((PAGE, D))
    kc = np.zeros((PAGE, D), np.int64)
    vc = np.zeros((PAGE, D), np.int64)
    half = np.arange(-7, 6) + 0.5                                   # -6.5 .. 5.5
    want = np.round(half).astype(np.int64)                         # numpy rounds half to even
    assert list(want[:4]) == [-6, -6, -4, -4]
    for d in range(D):
        vals = np.concatenate([[-8.0, 7.0], np.resize(np.roll(half, d), PAGE - 2)])
        K[:, d] = vals
        kc[:, d] = np.concatenate([[-8, 7], np.resize(np.roll(want, d), PAGE - 2)])
    for t in range(PAGE):
        vals = np.concatenate([[-8.0, 7.0], np.resize(np.roll(half, t), D - 2)])
        V[t] = vals
        vc[t] = np.concatenate([[-8, 7], np.resize(np.roll(want, t), D - 2)])
    ones, zeros_d, zeros_t = np.ones(D), np.zeros(D), np.zeros(PAGE)
    rec = record(kc, ones, zeros_d, vc, np.ones(PAGE), zeros_t, D, bits)
    return dict(K=K.astype(np.float32)[None], V=V.astype(np.float32)[None], rec=rec[None, None])


def const_case(rng, bits: int):
    D = 64
    H = 2 ** (bits - 1)
    ks, kb = dyadic_params(rng, D, bits)
    kc = codes_with_extremes(rng, (PAGE, D), 0, bits)
    vs, vb = dyadic_params(rng, PAGE, bits)
    vc = codes_with_extremes(rng, (PAGE, D), 1, bits)
    K = kb[None, :] + kc * ks[None, :]
    V = vb[:, None] + vc * vs[:, None]
    K[:, 5] = np.float32(0.1)                                       # constant channel
    ks[5], kb[5], kc[:, 5] = 0.0, np.float16(np.float32(0.1)), 0
    V[7, :] = np.float32(-0.3)                                      # constant row
    vs[7], vb[7], vc[7, :] = 0.0, np.float16(np.float32(-0.3)), 0
    assert H > 0
    rec = record(kc, ks, kb, vc, vs, vb, D, bits)
    return dict(K=K.astype(np.float32)[None], V=V.astype(np.float32)[None], rec=rec[None, None])


def clamp_case(rng):
    D, bits = 64, 4
    ks, kb = dyadic_params(rng, D, bits)
    kc = codes_with_extremes(rng, (PAGE, D), 0, bits)
    vs, vb = dyadic_params(rng, PAGE, bits)
    vc = codes_with_extremes(rng, (PAGE, D), 1, bits)
    K = kb[None, :] + kc * ks[None, :]
    V = vb[:, None] + vc * vs[:, None]
    u = 2.0 ** -24
    k = np.concatenate([np.arange(17), [16.5], np.arange(14)])      # 32 values, min 0, max 16.5
    K[:, 9] = k * u
    assert np.float16(np.float32(16.5 * u / 15)) == np.float16(u)   # the fp16 scale is the subnormal 2^-24
    ks[9], kb[9] = u, 8 * u
    kc[:, 9] = np.clip(np.round(k - 8), -8, 7)
    assert kc[16, 9] == 7 and kc[17, 9] == 7 and kc[0, 9] == -8
    rec = record(kc, ks, kb, vc, vs, vb, D, bits)
    return dict(K=K.astype(np.float32)[None], V=V.astype(np.float32)[None], rec=rec[None, None])


def main() -> None:
    rng = np.random.default_rng(0)
    arrays = {}
    for D in (64, 128):
        for bits in (4, 8):
            for key, val in exact_case(rng, D, bits).items():
                arrays[f"exact_D{D}_b{bits}_{key}"] = val
    for key, val in ties_case().items():
        arrays[f"ties_D64_b4_{key}"] = val
    for bits in (4, 8):
        for key, val in const_case(rng, bits).items():
            arrays[f"const_D64_b{bits}_{key}"] = val
    for key, val in clamp_case(rng).items():
        arrays[f"clamp_D64_b4_{key}"] = val
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
