"""Independent writer of .qwenbin v2 test containers, following the
reference's exporter (tools/export_qwen25.py:218-419): header struct
'<12I2f2I11Q' in a 4096-byte page, LayerDescriptor '<2I26Q' (216 bytes) from
offset 4096, payload from the next 256-byte boundary, every tensor padded to
256 bytes, tensors in the exporter's order.  Used by the loader tests to
check the reader against the format's own description, not against the
library's writer."""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x5157454E
HEADER_FMT = "<12I2f2I11Q"
LAYER_FMT = "<2I26Q"


def center_nibbles(w: np.ndarray) -> np.ndarray:
    """Every zero nibble of the packed words becomes 8: uniform nibbles in
    [0, 15] then have mean exactly 8 (the zero point), i.e. weights with no
    common-mode term."""
    t = w | (w >> 1)
    t |= t >> 2
    zero = ~t & np.uint32(0x11111111)  # bit 0 of each nibble that is 0
    return w | (zero << 3)


def synth_model(L=2, H=256, I=256, nq=2, nkv=1, V=512, seed=0, untied=False, centered=False):
    """Random tensors of a small GQA model in the packed W4A16 G128 layout.
    centered: layer weights with nibble mean 8 (center_nibbles), scales
    |N(0,1)| / sqrt(17.5 K) (the variance of such a weight is 17.5 s^2)."""
    rng = np.random.default_rng(seed)
    qd, kvd = nq * 128, nkv * 128

    def mat(N, K):
        if centered:
            w = center_nibbles(np.frombuffer(rng.bytes(N * K // 2), np.uint32).reshape(N, K // 8))
            s = (np.abs(rng.standard_normal((N, K // 128))) / np.sqrt(17.5 * K)).astype(np.float16)
            return w, s
        w = rng.integers(0, 2 ** 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
        s = (np.abs(rng.standard_normal((N, K // 128))) / np.sqrt(21.5 * K)).astype(np.float16)
        return w, s

    def vec(n, mean=0.0, std=0.02):
        return (mean + std * rng.standard_normal(n)).astype(np.float16)

    m = {"dims": dict(L=L, H=H, I=I, nq=nq, nkv=nkv, V=V)}
    m["embed"] = mat(V, H)
    m["embed"] = (m["embed"][0], (np.abs(rng.standard_normal((V, H // 128))) * 0.02).astype(np.float16))
    m["lm_head"] = mat(V, H) if untied else None
    m["final_norm"] = vec(H, 1.0, 0.05)
    m["layers"] = []
    for _ in range(L):
        m["layers"].append(dict(ln1=vec(H, 1.0, 0.05), q=mat(qd, H), k=mat(kvd, H), v=mat(kvd, H), q_b=vec(qd),
                                k_b=vec(kvd), v_b=vec(kvd), o=mat(H, qd), ln2=vec(H, 1.0, 0.05),
                                gu=mat(2 * I, H), dn=mat(H, I)))
    return m


def write(path, m, max_seq_len=1024, rope_theta=1e6, quant=1, version=2, layer_type=0, mutate=None):
    d = m["dims"]
    L = d["L"]
    table = 4096
    wofs = (table + L * 216 + 255) & ~255
    payload = bytearray()

    def put(arr) -> int:
        off = wofs + len(payload)
        payload.extend(np.ascontiguousarray(arr).tobytes())
        payload.extend(b"\0" * ((-len(payload)) % 256))
        return off

    ew = put(m["embed"][0])
    es = put(m["embed"][1])
    if m["lm_head"] is not None:
        lw, ls = put(m["lm_head"][0]), put(m["lm_head"][1])
    else:
        lw, ls = ew, 0
    fn = put(m["final_norm"])
    descs = []
    for t in m["layers"]:
        n1 = put(t["ln1"])
        qo, qs = put(t["q"][0]), put(t["q"][1])
        ko, ks = put(t["k"][0]), put(t["k"][1])
        vo, vs = put(t["v"][0]), put(t["v"][1])
        qb, kb, vb = put(t["q_b"]), put(t["k_b"]), put(t["v_b"])
        oo, os_ = put(t["o"][0]), put(t["o"][1])
        n2 = put(t["ln2"])
        gu, gs = put(t["gu"][0]), put(t["gu"][1])
        dn, ds = put(t["dn"][0]), put(t["dn"][1])
        descs.append([layer_type, 0, n1, n2, qo, qb, kb, vb, oo, 0, 0, 0, 0, 0, gu, gu, dn, qs, 0, ko, vo, qs, ks, vs,
                      os_, gs, gs, ds])
    hdr = [MAGIC, version, d["H"], d["I"], L, d["nq"], d["nkv"], 128, d["V"], max_seq_len, quant,
           0 if m["lm_head"] is not None else 1, 1e-6, rope_theta, 0, 0, table, ew, fn, lw, wofs, es, ls, 0, 0, 0, 0]
    if mutate:
        mutate(hdr, descs)
    blob = bytearray(wofs)
    struct.pack_into(HEADER_FMT, blob, 0, *hdr)
    for l, dsc in enumerate(descs):
        struct.pack_into(LAYER_FMT, blob, table + 216 * l, *dsc)
    with open(path, "wb") as f:
        f.write(blob)
        f.write(payload)
    return {"weights_offset": wofs, "size": wofs + len(payload), "header": hdr, "descs": descs}
