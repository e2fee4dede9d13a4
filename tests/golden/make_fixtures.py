"""Writes tests/golden/fixtures.json -- known-answer vectors for the oracle.

Nothing here runs or imports the reference (it is Rust; no toolchain).  The
vectors come from:
  * the reference's own test fixtures, restated: make_q4k_block / make_weight
    / make_x (swamp-kernels/src/fused_gemv_q4k.rs:708-740) and the xorshift64
    int8 stream of the VNNI test (swamp-kernels/src/lib.rs:600-606), with
    expected values from closed forms evaluated in float64 / exact integers;
  * hand-written known answers for the block layouts the reference's scalar
    dequantizers read (q4_0.rs:30-35 interleaved nibbles; q4_k.rs:290-319
    layout A), written out literally below;
  * a Q6_K block built by a packer written from the published layout (the
    inverse direction of q6_k.rs:36-44), and the reference's Q6_K GEMV test
    data create_test_data (fused_gemv_q6k.rs:329-357) with its values read
    back through the same layout.
Run:  python tests/golden/make_fixtures.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_bytes(v):
    return list(np.array([v], dtype=np.float32).astype(np.float16).tobytes())


def make_q4k_block(d, dmin, scales, mins, nibble_val):
    # fused_gemv_q4k.rs:708-724
    b = [0] * 144
    b[0:2] = f16_bytes(d)
    b[2:4] = f16_bytes(dmin)
    for j in range(4):
        b[4 + j] = (scales[j] & 0x3F) | ((scales[4 + j] >> 4) << 6)
        b[8 + j] = (mins[j] & 0x3F) | ((mins[4 + j] >> 4) << 6)
    for j in range(4):
        b[12 + j] = (scales[4 + j] & 0x0F) | ((mins[4 + j] & 0x0F) << 4)
    for i in range(128):
        b[16 + i] = nibble_val | (nibble_val << 4)
    return b


def make_weight(n_rows):
    # fused_gemv_q4k.rs:726-736 (one 256-weight block per row)
    w, rows = [], []
    for r in range(n_rows):
        d = np.float32(0.5) + np.float32(r) * np.float32(0.1)
        dm = np.float32(0.1) + np.float32(r) * np.float32(0.05)
        sc = (r + 1) & 0x3F
        mn = (r + 2) & 0x3F
        w += make_q4k_block(float(d), float(dm), [sc] * 8, [mn] * 8, 8)
        rows.append((float(np.float32(d).astype(np.float16)), float(np.float32(dm).astype(np.float16)), sc, mn))
    return w, rows


def make_x(n_cols):
    # fused_gemv_q4k.rs:738-740: (i % 100) as f32 / 50.0 - 1.0
    return [float(np.float32(np.float32(i % 100) / np.float32(50.0) - np.float32(1.0))) for i in range(n_cols)]


def gemv_closed_form(n_rows):
    """y_r = sum_j (8 d_r sc_r - dm_r mn_r) * sum_{i in sub-block j} x_i, f64."""
    w, rows = make_weight(n_rows)
    x = make_x(256)
    y = []
    for (d, dm, sc, mn) in rows:
        wv = 8.0 * d * sc - dm * mn
        y.append(wv * sum(x))
    return w, x, y, [8.0 * d * sc - dm * mn for (d, dm, sc, mn) in rows]


def xorshift_stream(seed, n):
    s = seed
    out = []
    m = (1 << 64) - 1
    for _ in range(n):
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        v = s & 0xFF
        out.append(v - 256 if v >= 128 else v)
    return out, s


def int8_dot_kat():
    # lib.rs:600-623: 32 trials, k = 64,128,192,256, w then acts per trial
    s = 0xDEAD_BEEF_1234_5678
    trials = []
    for trial in range(32):
        k = (trial % 4 + 1) * 64
        w, s = xorshift_stream(s, k)
        a, s = xorshift_stream(s, k)
        trials.append({"k": k, "w": w, "a": a, "dot": int(sum(int(p) * int(q) for p, q in zip(w, a)))})
    return trials


# ------------------------------------------------------------------ Q6_K
# Layout of a 210-byte Q6_K block as ggml publishes it and the reference's
# dequantizer reads it (swamp-gguf/src/quant/q6_k.rs:25-49): ql[128],
# qh[64], int8 sc[16], f16 d.  Element e (0..255) is in half h = e // 128,
# group k = (e % 128) // 32, column l = e % 32; its 6-bit code q has the low
# 4 bits in ql[64h + 32(k & 1) + l] (low nibble for k < 2, high for k >= 2)
# and bits 4-5 in qh[32h + l] bits 2k..2k+1; its scale is sc[e // 16]; its
# value is d * sc * (q - 32).

def q6k_pack(q, sc, d_code):
    """Block bytes for codes q[256] (0..63), int8 scales sc[16], f16 d."""
    b = [0] * 210
    for e, v in enumerate(q):
        h, k, l = e // 128, (e % 128) // 32, e % 32
        i = 64 * h + 32 * (k & 1) + l
        b[i] |= (v & 0xF) << (4 if k >= 2 else 0)
        b[128 + 32 * h + l] |= ((v >> 4) & 3) << (2 * k)
    for j in range(16):
        b[192 + j] = sc[j] & 0xFF
    b[208], b[209] = d_code & 0xFF, d_code >> 8
    return b


def q6k_codes(blk):
    """Inverse of q6k_pack: (q[256], sc[16], d_code) of a block."""
    q = []
    for e in range(256):
        h, k, l = e // 128, (e % 128) // 32, e % 32
        lo = blk[64 * h + 32 * (k & 1) + l]
        lo = (lo >> 4) if k >= 2 else (lo & 0xF)
        q.append(lo | (((blk[128 + 32 * h + l] >> (2 * k)) & 3) << 4))
    sc = [v - 256 if v >= 128 else v for v in blk[192:208]]
    return q, sc, blk[208] | (blk[209] << 8)


def q6k_create_test_data(n_rows, n_blocks):
    # the reference's fixture, fused_gemv_q6k.rs:329-357
    raw = []
    for row in range(n_rows):
        for _ in range(n_blocks):
            b = [0] * 210
            for i in range(128):
                b[i] = (i & 0x0F) | (((i + 128) & 0x0F) << 4)
            for i in range(64):
                b0 = (i >> 4) & 3
                b1 = ((i + 64) >> 4) & 3
                b2 = ((i + 128) >> 4) & 3
                b3 = ((i + 192) >> 4) & 3
                b[128 + i] = b0 | (b1 << 2) | (b2 << 4) | (b3 << 6)
            for i in range(16):
                b[192 + i] = (row * 16 + i + 1) & 0x7F
            b[208], b[209] = 0x00, 0x38  # d = 0.5
            raw += b
    return raw


def q6k_fixtures():
    out = {}
    # layout KAT: distinct codes, signed scales (-128 included), d = 1
    q = [(7 * e + 3) % 64 for e in range(256)]
    sc = [1, -2, 3, -4, 5, -6, 7, -8, 9, -10, 11, -12, 13, -14, 15, -128]
    blk = q6k_pack(q, sc, 0x3C00)
    assert q6k_codes(blk) == (q, sc, 0x3C00)
    out["q6_k_layout_kat"] = {"raw": blk, "q": q, "sc": sc,
                              "expected": [float(sc[e // 16] * (q[e] - 32)) for e in range(256)]}
    # the reference's GEMV test data, with its per-element values from the
    # layout above (exact: d = 0.5, small integers)
    fxs = []
    for n_rows, n_blocks in ((2, 2), (4, 3)):
        raw = q6k_create_test_data(n_rows, n_blocks)
        vals = []
        for r in range(n_rows):
            for b in range(n_blocks):
                off = (r * n_blocks + b) * 210
                qq, ss, dc = q6k_codes(raw[off:off + 210])
                assert dc == 0x3800
                vals += [0.5 * ss[e // 16] * (qq[e] - 32) for e in range(256)]
        fxs.append({"n_rows": n_rows, "n_blocks": n_blocks, "raw": raw, "w_values": vals})
    out["q6_k_reference_test_data"] = fxs
    return out


def main():
    fx = {}
    # Q4_0 interleave KAT (q4_0.rs:30-35): element 2j is the LOW nibble of
    # byte j, element 2j+1 the HIGH nibble; value nibble - 8.
    nib = [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE,
           0x01, 0x23, 0x45, 0x67, 0x89, 0xAB, 0xCD, 0xEF]
    blk1 = [0x00, 0x3C] + nib           # d = 1.0
    blk2 = [0x00, 0x38] + nib           # d = 0.5
    e = [-8, -7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 7,
         -7, -8, -5, -6, -3, -4, -1, -2, 1, 0, 3, 2, 5, 4, 7, 6]
    fx["q4_0_kat"] = {"raw": blk1 + blk2, "expected": e + [v * 0.5 for v in e]}
    # Q8_0: d = 1 is the int8 identity, d = 0.125 scales exactly.
    qs = list(range(-128, -96))
    fx["q8_0_kat"] = {"raw": [0x00, 0x3C] + [q & 0xFF for q in qs] + [0x00, 0x30] + [q & 0xFF for q in qs],
                      "expected": [float(q) for q in qs] + [q * 0.125 for q in qs]}
    # Q4_K layout A KAT: d = 1, dmin = 0, all scales 1, mins 0, nibble byte
    # k holds the value k (k = 0..127).  Layout A: sub-block 2p element i =
    # low nibble of byte 32p+i = i & 15; sub-block 2p+1 element i = high
    # nibble = 2p + (i >= 16).
    blk = make_q4k_block(1.0, 0.0, [1] * 8, [0] * 8, 0)
    for k in range(128):
        blk[16 + k] = k
    exp_a = []
    for p in range(4):
        exp_a += [float(i & 15) for i in range(32)]
        exp_a += [float(2 * p)] * 16 + [float(2 * p + 1)] * 16
    fx["q4_k_layout_kat"] = {"raw": blk, "expected": exp_a}
    # Q4_K scales/mins: block from the reference's packer with distinct codes;
    # every nibble 8 -> value 8*d*sc_j - dmin*m_j for sub-block j.
    sc = [1, 7, 13, 63, 32, 17, 40, 5]
    mn = [2, 0, 63, 9, 48, 33, 16, 60]
    blk = make_q4k_block(0.25, 0.125, sc, mn, 8)
    fx["q4_k_scale_kat"] = {"raw": blk, "scales": sc, "mins": mn,
                            "expected": [8 * 0.25 * sc[j] - 0.125 * mn[j] for j in range(8) for _ in range(32)]}
    # fused GEMV fixtures of the reference tests (rows 2,3,4,7) + closed form
    fx["gemv_fixtures"] = []
    for n_rows in (2, 3, 4, 7):
        w, x, y, wv = gemv_closed_form(n_rows)
        fx["gemv_fixtures"].append({"n_rows": n_rows, "w": w, "x": x, "y": y, "w_value": wv})
    fx["int8_dot_kat"] = int8_dot_kat()
    fx.update(q6k_fixtures())
    with open(os.path.join(HERE, "fixtures.json"), "w") as f:
        json.dump(fx, f)
    print("wrote", os.path.join(HERE, "fixtures.json"))


if __name__ == "__main__":
    main()
