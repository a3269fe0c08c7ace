"""Writes tests/golden/fixtures.npz: known-answer vectors for the fixed-mode
BF16 codec, computed by an encoder/decoder written here directly from the
stream description of the reference (integration/cuszp_wrapper/
cuszp_batched_fixed.cu) with numpy/torch arithmetic and per-bit loops.

This generator is independent of oracle/kvszp_oracle.c on purpose: the
fixtures then check the oracle (tests/test_golden.py, CPU) and the HIP codec
(the same file, GPU) against a second, deliberately naive restatement.

    python tests/golden/make_golden.py        # rewrites fixtures.npz

Arithmetic used (each a correctly-rounded library operation):
  * relative bound  eb = f32(eps) * max(f32(max - min), f32(1e-6))   cu:128-131
    over the logical values, NaN ignored (fmaxf/fminf, cu:78-79)
  * recip = f32(0.5) / eb                                             cu:166
  * v = f32(x * recip); s = 0 if v >= -0.5 else 1 (NaN -> 1)          cu:17-19
  * t = f32(v + 0.5)            (two roundings), or
    t = f32(x * recip + 0.5)    (fused: the exact value rounded once; x*recip
    of two f32 is exact in f64, and so is the +0.5 whenever |x*recip| >=
    2^-6; below that t lies in (0.48, 0.52) and truncates to 0 either way)
  * c = trunc(t) saturated to int32, NaN -> 0; q = int32(c - s) wrapping
  * rate = bit length of max |q| over the 32-element block            cu:27-31
  * header: R = 1024*ceil(n/32768) bytes, byte b = rate of block b, padding 0
  * payload per block with rate r > 0: sign word then r plane words; element v
    sits in byte v>>3 at bit 7-(v&7)                                  cu:320-351
  * decode y = bf16_rne(f32(f32(f32(q) * eb) * 2)), rate-0 blocks -> +0.0
"""

from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "fixtures.npz")
INT32_MIN, INT32_MAX = -(2**31), 2**31 - 1


def to_bf16(values) -> np.ndarray:
    t = torch.tensor(np.asarray(values, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def from_bf16(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def logical_values(page_bits, n, layers=None, src=0, epl=0):
    """The segment's values in logical order (index_select over layers)."""
    x = from_bf16(page_bits)
    if layers is None:
        return x[:n]
    view = x.reshape(-1, src, epl)
    return view[:, list(layers), :].reshape(-1)[:n]


def relative_bound(x: np.ndarray, eps: float) -> np.float32:
    finite = x[~np.isnan(x)]
    mx, mn = np.float32(finite.max()), np.float32(finite.min())
    rng = np.float32(mx - mn)
    return np.float32(np.float32(eps) * max(rng, np.float32(1e-6)))


def quantize(x: np.ndarray, recip: np.float32, fused: bool) -> np.ndarray:
    x = x.astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        v = (x * recip).astype(np.float32)
        s = np.where(v >= np.float32(-0.5), 0, 1).astype(np.int64)
        if fused:
            t = (x.astype(np.float64) * np.float64(recip) + 0.5).astype(np.float32)
        else:
            t = (v + np.float32(0.5)).astype(np.float32)
        c = np.zeros(len(x), dtype=np.int64)
        ok = ~np.isnan(t)
        tt = t[ok].astype(np.float64)
        c[ok] = np.where(tt >= 2.0**31, INT32_MAX,
                         np.where(tt <= -(2.0**31), INT32_MIN, np.trunc(tt))).astype(np.int64)
    q = c - s
    return ((q - INT32_MIN) % 2**32) + INT32_MIN


def encode(q: np.ndarray) -> bytes:
    n = len(q)
    nb = (n + 31) // 32
    R = 1024 * ((n + 32767) // 32768)
    header = bytearray(R)
    payload = bytearray()
    for b in range(nb):
        blk = [int(v) for v in q[32 * b:32 * b + 32]] + [0] * max(0, 32 * b + 32 - n)
        mags = [abs(v) for v in blk]
        rate = max(mags).bit_length()
        header[b] = rate
        if rate == 0:
            continue
        sign = bytearray(4)
        for v in range(32):
            if blk[v] < 0:
                sign[v >> 3] |= 1 << (7 - (v & 7))
        payload += sign
        for p in range(rate):
            plane = bytearray(4)
            for v in range(32):
                if (mags[v] >> p) & 1:
                    plane[v >> 3] |= 1 << (7 - (v & 7))
            payload += plane
    return bytes(header) + bytes(payload)


def decode(stream: bytes, n: int, eb: np.float32) -> np.ndarray:
    nb = (n + 31) // 32
    R = 1024 * ((n + 32767) // 32768)
    q = np.zeros(nb * 32, dtype=np.int64)
    pos = R
    for b in range(nb):
        rate = stream[b]
        if rate == 0:
            continue
        words = [stream[pos + 4 * k:pos + 4 * k + 4] for k in range(rate + 1)]
        pos += 4 * (rate + 1)
        for v in range(32):
            bit = lambda w: (w[v >> 3] >> (7 - (v & 7))) & 1
            m = sum(bit(words[1 + p]) << p for p in range(rate))
            q[32 * b + v] = -m if bit(words[0]) else m
    y = (q[:n].astype(np.float32) * eb).astype(np.float32) * np.float32(2.0)
    out = to_bf16(y.astype(np.float32))
    # rate-0 blocks decode to +0.0 (q = 0 gives +0.0 as well)
    return out


def kv_like(rng, n, outliers=True) -> np.ndarray:
    d = 128
    sigma = np.exp(0.5 * rng.standard_normal(d))
    if outliers:
        sigma[rng.choice(d, 4, replace=False)] *= 15.0
    z = rng.standard_normal(n)
    return to_bf16(z * np.resize(sigma, n))


def cases():
    rng = np.random.default_rng(20241201)
    out = []
    # plain pages, absolute and relative bounds
    out.append(dict(name="abs_small", page=to_bf16(rng.standard_normal(1000) * 3.0),
                    n=1000, eps=0.01, relative=0, fused=0))
    out.append(dict(name="rel_cross_ref_tile", page=kv_like(rng, 33000), n=33000,
                    eps=1e-4, relative=1, fused=0))
    x = from_bf16(kv_like(rng, 16401)).copy()
    x[64:192] = 0.0                  # four all-zero blocks (rate 0)
    x[300:340] = 2.5                 # a constant run
    x[1000] = np.nan                 # NaN: ignored by the bound, q = -1
    x[5000] = -0.0
    out.append(dict(name="rel_specials", page=to_bf16(x), n=16401, eps=1e-5,
                    relative=1, fused=0))
    # layer-indexed segment: page view(2, 5, 320), layers (3, 0, 4)
    out.append(dict(name="indexed", page=kv_like(rng, 2 * 5 * 320), n=2 * 3 * 320,
                    eps=1e-4, relative=1, fused=0, layers=(3, 0, 4), src=5, epl=320))
    # double-rounding inputs: the two quantizer readings disagree here
    page = to_bf16(rng.uniform(1.0, 2.0, 640) * rng.choice([-1.0, 1.0], 640))
    eb = float(np.float32(0.5) / np.float32(2.0**23 + 12345.0))
    for fused in (0, 1):
        out.append(dict(name=f"double_rounding_{'fused' if fused else 'two'}",
                        page=page, n=640, eps=eb, relative=0, fused=fused))
    return out


def main() -> None:
    arrays = {}
    names = []
    for c in cases():
        layers = c.get("layers")
        x = logical_values(c["page"], c["n"], layers, c.get("src", 0), c.get("epl", 0))
        eb = relative_bound(x, c["eps"]) if c["relative"] else np.float32(c["eps"])
        recip = np.float32(np.float32(0.5) / eb)
        q = quantize(x, recip, bool(c["fused"]))
        stream = encode(q)
        dec = decode(stream, c["n"], eb)
        k = c["name"]
        names.append(k)
        arrays[f"{k}.page"] = c["page"]
        arrays[f"{k}.params"] = np.array(
            [c["n"], c["relative"], c["fused"], c.get("src", 0), c.get("epl", 0)],
            dtype=np.int64)
        arrays[f"{k}.eps"] = np.array([c["eps"]], dtype=np.float32)
        arrays[f"{k}.layers"] = np.array(layers or (), dtype=np.int64)
        arrays[f"{k}.eb"] = np.array([eb], dtype=np.float32)
        arrays[f"{k}.stream"] = np.frombuffer(stream, dtype=np.uint8)
        arrays[f"{k}.decoded"] = dec
    arrays["cases"] = np.array(names)
    np.savez_compressed(OUT, **arrays)
    print("wrote", OUT, os.path.getsize(OUT), "bytes,", len(names), "cases")


if __name__ == "__main__":
    main()
