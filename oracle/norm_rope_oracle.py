"""CPU restatement of the attention prologue: per-head RMSNorm of q and k,
rotary embedding, and (through ``fp8_oracle.store_fp8_kvcache``) the FP8
store (test infrastructure).

Only the tests, ``__graft_entry__.smoke()`` and the benchmark's CPU baseline
may use this module, and only as the checker.  The product path is
``microserve_amd.qk_norm_rope`` over the HIP kernel
``qk_norm_rope_store_kernel``.

* ``rope_tables``  -- ``RotaryEmbedding.__init__``,
  ``microserve/layers/rotary_embedding.py:13-22``, then the runner's cast of
  the model (buffers included) to the activation type,
  ``microserve/engine/model_runner.py:58-59``.
* ``rms_norm``     -- ``RMSNorm.forward`` without residual on a strided head
  view (``microserve/layers/layernorm.py:55-57, 80-81``):
  ``T(T(x * rsqrt(mean(x^2) + eps)) * w)``.  torch leaves the fp32
  reduction order and the rounding of rsqrt unspecified; here they are fixed
  to the kernel's: lane l of 8 sums the squares of elements
  [8l, 8l+8) then [64+8l, 64+8l+8) in order, the 8 partial sums combine as
  ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7)), and rsqrt is 1/sqrt with both
  operations IEEE-rounded in fp32.
* ``rope``         -- ``RotaryEmbedding.forward``,
  ``rotary_embedding.py:24-31`` with ``rotate_half`` (:4-7), as torch CPU
  ops in the activation type (each product and the sum rounded to it, the
  sum in fp32 first).

Pinned by ``tests/test_norm_rope_oracle.py``: against the reference's own
formulation (``torch.rsqrt`` and ``mean``) to within one unit in the last
place on a small fraction of elements, closed forms (rows of equal
magnitude normalize to exactly +-w; position 0 leaves a row unchanged), and
the rotation against float64 trigonometry.
"""

from __future__ import annotations

import numpy as np
import torch

HEAD_DIM = 128


def rope_tables(max_position: int, base: float, dtype, head_dim: int = HEAD_DIM):
    """cos/sin tables [max_position, head_dim] in ``dtype``
    (rotary_embedding.py:16-22 computes them in fp32, the runner casts)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(max_position, dtype=torch.float32)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _lane_order(d: int = HEAD_DIM) -> np.ndarray:
    half = d // 2
    return np.concatenate([np.r_[8 * l:8 * l + 8, half + 8 * l:half + 8 * l + 8]
                           for l in range(8)])


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """x: [..., 128] in fp16/bf16, w: [128] in the same type."""
    dtype = x.dtype
    xf = x.float().reshape(-1, HEAD_DIM).numpy()
    lanes = xf[:, _lane_order()].reshape(-1, 8, 16)
    s = np.zeros(lanes.shape[:2], np.float32)
    with np.errstate(over="ignore"):  # fp32 squares of huge rows overflow to inf, as IEEE does
        for i in range(16):
            s = s + lanes[:, :, i] * lanes[:, :, i]
    tot = ((s[:, 0] + s[:, 1]) + (s[:, 2] + s[:, 3])) + ((s[:, 4] + s[:, 5]) + (s[:, 6] + s[:, 7]))
    var = tot / np.float32(HEAD_DIM)
    r = np.float32(1.0) / np.sqrt(var + np.float32(eps))
    n = torch.from_numpy((xf * r[:, None]).astype(np.float32)).to(dtype)
    y = (n.float() * w.float()).to(dtype)
    return y.reshape(x.shape)


def rms_norm_reference_formula(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """The reference's own expression (layernorm.py:55-57, 80-81) in torch CPU
    ops, for pinning ``rms_norm``."""
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    return (xf * torch.rsqrt(var + eps)).to(x.dtype) * w


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         positions: torch.Tensor) -> torch.Tensor:
    """x: [T, H, 128]; cos/sin: [max_position, 128] in x's type."""
    c = cos[positions].unsqueeze(1)
    s = sin[positions].unsqueeze(1)
    x1, x2 = x.chunk(2, dim=-1)
    rot = torch.cat((-x2, x1), dim=-1)
    return (x * c) + (rot * s)


def qk_norm_rope(q, k, positions, q_w, k_w, eps, cos, sin):
    """The prologue of microserve/models/qwen3.py:49-53 on CPU tensors;
    weights None means no norm (the qkv-bias models)."""
    if q_w is not None:
        q = rms_norm(q, q_w, eps)
        k = rms_norm(k, k_w, eps)
    return rope(q, cos, sin, positions), rope(k, cos, sin, positions)
