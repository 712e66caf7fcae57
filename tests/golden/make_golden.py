"""Writes the committed golden vectors under tests/golden/.

Run from the repository root:  python tests/golden/make_golden.py

* ``division_rows.json`` -- fp16/bf16 rows where the per-element quantizer
  ``e4m3fn(clamp(x / s))`` gives a different byte from the reciprocal form
  ``x * (1 / s)``.  The expected byte is computed with torch's CPU ops (the
  formula of ``tests/test_fp8.py:25-26`` / ``fp8_kv_cache.py:24-27``), not
  with the oracle, so the fixture checks the oracle as well as the kernel.
* ``ref_shapes.npz`` -- the two known-answer cases of the reference's kernel
  test (``tests/test_fp8_kv_attention.py:39-108``), with inputs drawn by
  ``cases.py`` from a seeded CPU generator (the reference draws on the CUDA
  RNG, which cannot be reproduced here).  It holds SHA-256 digests of the
  inputs and of the filled caches plus the float32 attention outputs, all
  computed with torch-CPU ops independently of the oracle.
"""

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import cases  # noqa: E402

BLOCK = 256
QH, KVH, D = 16, 8, 128
SCALE = D ** -0.5


def _torch_quant(x: torch.Tensor):
    s = x.float().abs().amax(-1).clamp_min(1e-8) / 448
    q = (x.float() / s[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), s


def division_rows():
    rows = []
    for name, dt in (("bfloat16", torch.bfloat16), ("float16", torch.float16)):
        g = torch.Generator().manual_seed(7)
        found = 0
        while found < 6:
            amax = (torch.rand(4096, generator=g) * 7.5 + 0.5).to(dt)
            x = ((torch.rand(4096, 64, generator=g) * 2 - 1) * amax.float()[:, None]).to(dt)
            x = torch.where(x.float().abs() > amax.float()[:, None], torch.zeros_like(x), x)
            row = torch.cat([amax[:, None], x], 1)
            q, s = _torch_quant(row)
            recip = (row.float() * (1.0 / s)[:, None]).clamp(-448, 448).to(
                torch.float8_e4m3fn).view(torch.uint8)
            bad = (recip != q).nonzero()
            for r, c in bad.tolist():
                if c == 0:
                    continue
                vals = torch.zeros(D, dtype=dt)
                vals[0] = row[r, 0]
                vals[1] = row[r, c]
                qq, ss = _torch_quant(vals[None])
                rows.append({"dtype": name,
                             "bits": vals.view(torch.int16).tolist(),
                             "bytes": qq[0].tolist(),
                             "scale_bits": int(ss.view(torch.int32)[0]),
                             "reciprocal_byte": int(recip[r, c])})
                found += 1
                if found >= 6:
                    break
    with open(os.path.join(HERE, "division_rows.json"), "w") as f:
        json.dump(rows, f)


def _gather(cache_u8, scales, table, length):
    rows = []
    for p in range(length):
        blk, off = int(table[p // BLOCK]), p % BLOCK
        rows.append(cache_u8[blk, off].view(torch.float8_e4m3fn).float()
                    * scales[blk, off, :, None])
    return torch.stack(rows)


def _store(key, value, kc, vc, ks, vs, slots):
    kq, ksc = _torch_quant(key)
    vq, vsc = _torch_quant(value)
    kc.view(-1, KVH, D)[slots] = kq
    vc.view(-1, KVH, D)[slots] = vq
    ks.view(-1, KVH)[slots] = ksc
    vs.view(-1, KVH)[slots] = vsc


def _digest(*tensors):
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def ref_shapes():
    out = {}
    head_map = torch.arange(QH) // (QH // KVH)
    c = cases.decode_case()
    kc = torch.zeros(c["num_blocks"], BLOCK, KVH, D, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    ks = torch.ones(c["num_blocks"], BLOCK, KVH)
    vs = torch.ones_like(ks)
    _store(c["key"], c["value"], kc, vc, ks, vs, c["slots"])
    refs = []
    for b, n in enumerate(c["lengths"]):
        k = _gather(kc, ks, c["tables"][b], n)[:, head_map]
        v = _gather(vc, vs, c["tables"][b], n)[:, head_map]
        sc = torch.einsum("hd,lhd->hl", c["query"][b].float(), k) * SCALE
        refs.append(torch.einsum("hl,lhd->hd", sc.softmax(-1), v))
    out.update(dec_inputs=_digest(c["key"], c["value"], c["query"]),
               dec_cache=_digest(kc, vc, ks, vs),
               dec_out=torch.stack(refs).numpy())
    c = cases.chunk_case()
    kc = torch.zeros(c["num_blocks"], BLOCK, KVH, D, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    ks = torch.ones(c["num_blocks"], BLOCK, KVH)
    vs = torch.ones_like(ks)
    _store(c["key"], c["value"], kc, vc, ks, vs, c["slots"])
    prefix, lq = c["prefix"], c["query"].shape[0]
    k = _gather(kc, ks, c["table"][0], prefix + lq)[:, head_map]
    v = _gather(vc, vs, c["table"][0], prefix + lq)[:, head_map]
    refs = []
    for i in range(lq):
        vis = prefix + i + 1
        sc = torch.einsum("hd,lhd->hl", c["query"][i].float(), k[:vis]) * SCALE
        refs.append(torch.einsum("hl,lhd->hd", sc.softmax(-1), v[:vis]))
    out.update(pre_inputs=_digest(c["key"], c["value"], c["query"]),
               pre_cache=_digest(kc, vc, ks, vs),
               pre_out=torch.stack(refs).numpy())
    np.savez_compressed(os.path.join(HERE, "ref_shapes.npz"), **out)


if __name__ == "__main__":
    division_rows()
    ref_shapes()
    print("wrote", os.listdir(HERE))
