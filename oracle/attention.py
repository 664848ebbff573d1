"""CPU oracle for nemotron_infer's attention (decode and prefill) -- TEST INFRASTRUCTURE ONLY.

Restates on the CPU what the reference's attention computes, so that the HIP kernels
can be checked against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it.  bf16 tensors are uint16 bit patterns, as in ``oracle.linear``.

* ``sdpa_decode`` -- ops/attention/sdpa_decode.cuh:57-166 (split + combine kernels) and the CPU
  reference of tests/ops/test_sdpa_decode.cu:20-44: for every query head h,
  o[h] = softmax(q[h] . K[kv(h), 0:S]^T / sqrt(D)) . V[kv(h), 0:S] with
  kv(h) = h // (H / H_KV) (sdpa_decode.cuh:93), over the S cached positions only -- the new
  token's K/V are appended after the attention (sdpa_decode.cuh:160-174; the reference's test
  leaves them out of the expectation, test_sdpa_decode.cu:103-104).  S == 0 gives 0 (the
  combine's ``gl > 0`` branch, sdpa_decode.cuh:152).  Computed in float64 and rounded once to
  bf16: the reference and the kernel both work in float32, each in its own order; the float64
  value is what both approximate.
* ``append_kv`` -- the cache update of sdpa_decode.cuh:160-174: K[kv, S] = k_new[kv],
  V[kv, S] = v_new[kv]; every other position unchanged.
* ``attn_decode_block_fp8`` -- model/attention_block.cuh:371-414: h = rmsnorm(input) (bf16),
  q, k_new, v_new = fp8 linears of h (bf16 outputs), o = sdpa_decode(q, caches, S) (bf16),
  out = bf16(input + bf16(o_proj(o))); returns out and the updated caches.  NoPE (no rotary;
  attention_block.cuh:8-10).  The projections are ``oracle.linear``'s; the RMSNorm and the add
  are ``oracle.block``'s.
* ``sdpa_prefill`` -- ops/attention/sdpa_prefill.cuh:224-320: causal attention of every query
  s over keys t <= s of its KV head, float64, rounded once to bf16; token-major q [S, H*D],
  k, v [S, H_KV*D].
* ``attn_forward_block_fp8`` -- model/attention_block.cuh:289-366 on bf16 activations (the
  reference's e4m3 activation quantization into its GEMMs is not reproduced, as for every
  linear of this build): rmsnorm -> q, k, v linears -> sdpa_prefill -> o linear -> residual
  add; k and v are what the reference copies into the caches (:355-364).

Pinned in tests/test_oracle_attention.py: ``sdpa_decode`` against torch's own
``F.scaled_dot_product_attention`` in float64 with the KV heads repeated (a library routine,
independent of this restatement), against closed forms (one cached position returns V exactly;
a zero query returns the mean of V; S == 0 returns 0) and with planted mistakes (a wrong KV-head
mapping, attending the new token, a dropped 1/sqrt(D)) that those checks catch; the block
against an independent float32 torch composition and against the closed forms o_w == 0 and
S == 0 (both give out == input).  ``sdpa_prefill`` against torch's scaled_dot_product_attention
with is_causal=True in float64 and the closed form of its first row (the value of position 0);
a non-causal variant is caught.
"""
from __future__ import annotations

import numpy as np

from . import block, linear

HEAD = 128


def _f64(bits: np.ndarray) -> np.ndarray:
    return linear.bf16_to_f32(np.asarray(bits, np.uint16)).astype(np.float64)


def sdpa_decode_f64(q_bits, k_cache_bits, v_cache_bits, S: int, kv_of=None) -> np.ndarray:
    """float64 o [H, D] before rounding.  q [H, D]; caches [H_KV, cap, D] (bf16 bits).
    ``kv_of(h, H, H_KV)`` maps a query head to its KV head (default h // (H / H_KV))."""
    q = _f64(q_bits)
    K = _f64(k_cache_bits)
    V = _f64(v_cache_bits)
    H, D = q.shape
    H_KV = K.shape[0]
    if kv_of is None:
        kv_of = lambda h, H, H_KV: h // (H // H_KV)  # noqa: E731
    out = np.zeros((H, D), np.float64)
    if S == 0:
        return out
    for h in range(H):
        kv = kv_of(h, H, H_KV)
        sc = (K[kv, :S] @ q[h]) / np.sqrt(D)
        p = np.exp(sc - sc.max())
        out[h] = (p @ V[kv, :S]) / p.sum()
    return out


def sdpa_decode(q_bits, k_cache_bits, v_cache_bits, S: int) -> np.ndarray:
    """o [H, D] bf16 bits (see the module docstring)."""
    return block.bf16_round_exact(sdpa_decode_f64(q_bits, k_cache_bits, v_cache_bits, S))


def append_kv(k_cache_bits, v_cache_bits, k_new_bits, v_new_bits, S: int):
    """Copies of the caches with position S of every KV head set to k_new / v_new."""
    kc = np.array(k_cache_bits, np.uint16, copy=True)
    vc = np.array(v_cache_bits, np.uint16, copy=True)
    H_KV = kc.shape[0]
    kc[:, S] = np.asarray(k_new_bits, np.uint16).reshape(H_KV, -1)
    vc[:, S] = np.asarray(v_new_bits, np.uint16).reshape(H_KV, -1)
    return kc, vc


def attn_decode_block_fp8(x_bits, norm_w, q_codes, q_s, k_codes, k_s, v_codes, v_s, o_codes, o_s,
                          k_cache_bits, v_cache_bits, S: int, n_kv: int, eps: float = 1e-5,
                          return_stages: bool = False):
    """The block at decode.  x [1, hidden] bf16 bits; weights e4m3 codes [rows, cols] with
    float32 per-row scales; caches [n_kv, cap, 128] bf16 bits.  Returns (out, k_cache, v_cache)
    (+ the stages)."""
    x_bits = np.atleast_2d(np.asarray(x_bits, np.uint16))
    h = block.rmsnorm_bf16(x_bits, norm_w, eps)
    q = linear.linear_fp8_w8a16(h, q_codes, q_s)
    kn = linear.linear_fp8_w8a16(h, k_codes, k_s)
    vn = linear.linear_fp8_w8a16(h, v_codes, v_s)
    H = q.shape[1] // HEAD
    o = sdpa_decode(q.reshape(H, HEAD), k_cache_bits, v_cache_bits, S)
    attn = linear.linear_fp8_w8a16(o.reshape(1, -1), o_codes, o_s)
    out = block.add_bf16(x_bits, attn)
    kc, vc = append_kv(k_cache_bits, v_cache_bits, kn.reshape(n_kv, HEAD), vn.reshape(n_kv, HEAD), S)
    if return_stages:
        return out, kc, vc, dict(normed=h, q=q, k_new=kn, v_new=vn, o=o, attn=attn)
    return out, kc, vc


def sdpa_prefill_f64(q_bits, k_bits, v_bits, n_kv: int, causal: bool = True) -> np.ndarray:
    """float64 o [S, H*D] before rounding (token-major bf16 bits in)."""
    q = _f64(q_bits)
    K = _f64(k_bits)
    V = _f64(v_bits)
    S = q.shape[0]
    H = q.shape[1] // HEAD
    r = H // n_kv
    out = np.zeros((S, H * HEAD), np.float64)
    mask = np.tril(np.ones((S, S), bool)) if causal else np.ones((S, S), bool)
    for h in range(H):
        kv = h // r
        qh = q[:, h * HEAD:(h + 1) * HEAD]
        kh = K[:, kv * HEAD:(kv + 1) * HEAD]
        vh = V[:, kv * HEAD:(kv + 1) * HEAD]
        sc = (qh @ kh.T) / np.sqrt(HEAD)
        sc = np.where(mask, sc, -np.inf)
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        out[:, h * HEAD:(h + 1) * HEAD] = (p @ vh) / p.sum(axis=1, keepdims=True)
    return out


def sdpa_prefill(q_bits, k_bits, v_bits, n_kv: int) -> np.ndarray:
    return block.bf16_round_exact(sdpa_prefill_f64(q_bits, k_bits, v_bits, n_kv))


def attn_forward_block_fp8(x_bits, norm_w, q_codes, q_s, k_codes, k_s, v_codes, v_s, o_codes, o_s, n_kv: int,
                           eps: float = 1e-5, return_stages: bool = False):
    """The block over a prompt: x [S, hidden] bf16 bits.  Returns out (+ the stages, whose k and
    v are the cache contents)."""
    x_bits = np.atleast_2d(np.asarray(x_bits, np.uint16))
    h = block.rmsnorm_bf16(x_bits, norm_w, eps)
    q = linear.linear_fp8_w8a16(h, q_codes, q_s)
    k = linear.linear_fp8_w8a16(h, k_codes, k_s)
    v = linear.linear_fp8_w8a16(h, v_codes, v_s)
    o = sdpa_prefill(q, k, v, n_kv)
    attn = linear.linear_fp8_w8a16(o, o_codes, o_s)
    out = block.add_bf16(x_bits, attn)
    if return_stages:
        return out, dict(normed=h, q=q, k=k, v=v, o=o, attn=attn)
    return out
