"""Offline INT4 weight packing and the packed formats (CPU, torch).

API mirror of the reference's ``pi05_fast/w4a4/pack.py``: the same function names,
argument meanings and on-disk/in-memory formats (Hadamard on K in {1024, 2048, 16384},
INT4 codes in [-7, 7], ``[N, K/8+1]`` int32 rows with the fp32 scale bits in word K/8).
Adds the gfx950 MFMA-fragment-major layout (``pack_mfma_weight`` /
``unpack_mfma_weight``) so weights can be packed straight into the layout the MI355X
kernels read.

Everything here is offline / CPU code.  The GPU ops never call into this module.
``quant_activation_cpu`` and ``int4_gemm_ref`` are the reference's exported CPU
reference functions, kept for API compatibility.
"""

from __future__ import annotations

import math
from typing import Any

import torch

ROTATE_K = frozenset({1024, 2048, 16384})
WMMA_PRESHUFFLE_PAD_WORDS = 9
MFMA_MARKER_WORDS = 16


def fwht_unnormalized(x: torch.Tensor) -> torch.Tensor:
    """Unnormalised Sylvester Walsh-Hadamard transform along the last dim (pack.py:18-31).

    Radix-2 stages of stride h = 1, 2, 4, ...; each stage maps the pair (i, i+h) with bit
    h of i clear to (a + b, a - b).
    """
    n = x.shape[-1]
    if n <= 0 or (n & (n - 1)) != 0:
        raise ValueError(f"FWHT length must be a power of 2, got {n}")
    lead = x.shape[:-1]
    y = x.contiguous().clone()
    h = 1
    while h < n:
        pairs = y.view(*lead, n // (2 * h), 2, h)
        lo, hi = pairs.unbind(dim=-2)
        y = torch.stack((lo + hi, lo - hi), dim=-2).reshape(*lead, n)
        h *= 2
    return y


def pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """codes [..., K] in [-8, 7] -> int32 [..., K/8]; element 8p+j in bits 4j..4j+3 (pack.py:34-42)."""
    if q.shape[-1] % 8 != 0:
        raise ValueError(f"K must be a multiple of 8, got {q.shape[-1]}")
    nib = (q.to(torch.int32) & 0xF).view(*q.shape[:-1], q.shape[-1] // 8, 8)
    word = torch.zeros(nib.shape[:-1], dtype=torch.int32, device=nib.device)
    for j in range(8):
        word = word | (nib[..., j] << (4 * j))
    return word


def unpack_nibbles(packed: torch.Tensor, k: int) -> torch.Tensor:
    """int32 [..., K/8] -> int32 codes [..., K]; nibble >= 8 is value - 16 (pack.py:71-76)."""
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=packed.device)
    nib = (packed.to(torch.int32).unsqueeze(-1) >> shifts) & 0xF
    q = torch.where(nib >= 8, nib - 16, nib)
    return q.reshape(*packed.shape[:-1], k)


def should_rotate(k: int, rotate: bool | None = None) -> bool:
    """Rotation iff K in {1024, 2048, 16384} unless forced (pack.py:79-82)."""
    if rotate is not None:
        return bool(rotate)
    return k in ROTATE_K


def pack_linear_weight(weight: torch.Tensor, rotate: bool | None = None) -> torch.Tensor:
    """Linear.weight [N, K] -> int32 [N, K/8+1] (pack.py:85-101).

    W' = FWHT(W) * fp32(1/sqrt(K)) when rotating; s = max(amax(|W'|), 1e-12) / 7;
    codes = clamp(round_half_even(W' / s), -7, 7); word K/8 holds the fp32 bits of s.
    """
    if weight.dim() != 2:
        raise ValueError(f"expected 2D weight, got {tuple(weight.shape)}")
    n, k = weight.shape
    if k % 64 != 0:
        raise ValueError(f"K must be a multiple of 64 for gemm_iu4, got {k}")
    w = weight.detach().to(device="cpu", dtype=torch.float32)
    if should_rotate(k, rotate):
        w = fwht_unnormalized(w) * (1.0 / math.sqrt(k))
    scale = w.abs().amax(dim=-1).clamp_min(1e-12) / 7.0
    codes = torch.round(w / scale[:, None]).clamp(-7, 7).to(torch.int32)
    return torch.cat([pack_nibbles(codes), scale.contiguous().view(torch.int32)[:, None]], dim=1)


def unpack_linear_weight(packed: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, int]:
    """int32 [N, K/8+1] -> (codes [N, K], scale fp32 [N], K) (pack.py:104-110)."""
    _, row = packed.shape
    k = (row - 1) * 8
    codes = unpack_nibbles(packed[:, :-1], k)
    scale = packed[:, -1].contiguous().view(torch.float32)
    return codes, scale, k


def preshuffle_wmma_weight(packed: torch.Tensor, k: int) -> torch.Tensor:
    """Layout L3 (pack.py:45-68): flat[(t*N + n)*2 + h] = L1[n, 2t + h], then the N scales,
    in an int32 [N, K/8+9] tensor (the ninth pad word is the layout marker)."""
    if packed.dim() != 2:
        raise ValueError(f"expected 2D packed weight, got {tuple(packed.shape)}")
    n = packed.shape[0]
    words = k // 8
    if k % 16 != 0 or packed.shape[1] < words + 1:
        raise ValueError(f"invalid packed weight shape {tuple(packed.shape)} for K={k}")
    out = torch.zeros((n, words + WMMA_PRESHUFFLE_PAD_WORDS), dtype=packed.dtype, device=packed.device)
    flat = out.view(-1)
    flat[: n * words] = packed[:, :words].reshape(n, words // 2, 2).transpose(0, 1).reshape(-1)
    flat[n * words : n * words + n] = packed[:, words]
    return out


def fragment_word_index(lines: int, k: int, device: torch.device | str = "cpu") -> torch.Tensor:
    """Index map of the MFMA-fragment-major layout of packed INT4 codes, shared by the
    weights (line = output column) and the quantized activations (line = row).

    Returns int64 [lines, K/8]: row-major packed word (line, kw) -> word of the fragment
    buffer.  With KB = ceil(K/128), the 16-line block b and 128-deep k block t form one
    1 KB fragment at word (b*KB + t)*256 made of 64 16-byte slots: slot L holds codes
    32*(L//16) .. +31 of block t of line 16*b + L%16 (the 16 bytes lane L of an MFMA wave
    loads).
    """
    if k % 64 != 0:
        raise ValueError(f"K must be a multiple of 64, got {k}")
    kb128 = (k + 127) // 128
    r = torch.arange(lines, dtype=torch.int64, device=device)[:, None]
    kw = torch.arange(k // 8, dtype=torch.int64, device=device)[None, :]
    slot = (r & 15) + 16 * ((kw & 15) >> 2)
    return ((r >> 4) * kb128 + (kw >> 4)) * 256 + slot * 4 + (kw & 3)


def mfma_payload_words(n: int, k: int) -> int:
    """Payload words of an MFMA-layout weight (K padded to a multiple of 128)."""
    return n * ((k + 127) // 128) * 16


def mfma_word_permutation(n: int, k: int, device: torch.device | str = "cpu") -> torch.Tensor:
    """dst payload word -> L1 word index n*(K/8) + kw, or -1 for a zero pad word."""
    if n % 16 != 0 or k % 64 != 0:
        raise ValueError(f"MFMA layout needs N % 16 == 0 and K % 64 == 0, got N={n}, K={k}")
    idx = fragment_word_index(n, k, device).reshape(-1)
    perm = torch.full((mfma_payload_words(n, k),), -1, dtype=torch.int64, device=device)
    perm[idx] = torch.arange(idx.numel(), dtype=torch.int64, device=device)
    return perm


# Nibble encodings of the MFMA layouts.  Byte j of a packed word holds the codes of
# k = 2j and 2j+1.  The reference packs both in two's complement (k = 2j in the low
# nibble).  The MFMA layouts store one nibble of each byte in offset binary (code + 8) so
# that the GPU unpacks either operand with one AND per int8 word:
#   activations: low nibble = a[2j] + 8,  high nibble = a[2j+1] (two's complement)
#   weights:     high nibble = b[2j],     low nibble = b[2j+1] + 8
# The offsets add 128 * (sum of odd-k activation codes) per row and 128 * (sum of even-k
# weight codes) per column to the integer dot product; those sums, times -128, are stored
# after the activation codes (qcorr) and after the weight scales (wcorr).
_LO = 0x0F0F0F0F
_FLIP = 0x08080808


def _u32(words: torch.Tensor) -> torch.Tensor:
    return words.to(torch.int64) & 0xFFFFFFFF


def _i32(words: torch.Tensor) -> torch.Tensor:
    return torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)


def encode_weight_words(words: torch.Tensor) -> torch.Tensor:
    """Reference int32 code words -> the MFMA weight encoding (nibbles of each byte swapped,
    new low nibble in offset binary)."""
    u = _u32(words)
    return _i32(((u & _LO) << 4) | (((u >> 4) & _LO) ^ _FLIP))


def decode_weight_words(words: torch.Tensor) -> torch.Tensor:
    """Inverse of ``encode_weight_words``."""
    u = _u32(words)
    return _i32((((u & _LO) ^ _FLIP) << 4) | ((u >> 4) & _LO))


def flip_activation_words(words: torch.Tensor) -> torch.Tensor:
    """Reference code words <-> the MFMA activation encoding (its own inverse)."""
    return _i32(_u32(words) ^ _FLIP)


def pack_mfma_weight(packed: torch.Tensor, k: int | None = None) -> torch.Tensor:
    """L1/L2 packed weight -> MFMA-fragment-major int32 [N, K/8+16] (CPU/offline form of the
    device repack): encoded payload in ``fragment_word_index`` order (pad words 0), then the
    N fp32 scale words, then the N column corrections wcorr = -128 * (even-k code sum)."""
    n = packed.shape[0]
    if k is None:
        k = (packed.shape[1] - 1) * 8
    words = k // 8
    out = torch.zeros((n, words + MFMA_MARKER_WORDS), dtype=torch.int32, device=packed.device)
    flat = out.view(-1)
    idx = fragment_word_index(n, k, packed.device).reshape(-1)
    flat[idx] = encode_weight_words(packed[:, :words].contiguous()).view(-1)
    pw = mfma_payload_words(n, k)
    flat[pw : pw + n] = packed[:, words]
    codes = unpack_nibbles(packed[:, :words], k)
    flat[pw + n : pw + 2 * n] = (-128 * codes[:, 0::2].sum(dim=1)).to(torch.int32)
    return out


def unpack_mfma_weight(mfma: torch.Tensor, k: int) -> torch.Tensor:
    """Inverse of ``pack_mfma_weight``: MFMA layout -> L1 [N, K/8+1]."""
    n = mfma.shape[0]
    flat = mfma.contiguous().view(-1)
    idx = fragment_word_index(n, k, mfma.device)
    pw = mfma_payload_words(n, k)
    return torch.cat([decode_weight_words(flat[idx]), flat[pw : pw + n, None]], dim=1)


def mfma_weight_corrections(mfma: torch.Tensor, k: int) -> torch.Tensor:
    """The wcorr words [N] of an MFMA-layout weight."""
    n = mfma.shape[0]
    pw = mfma_payload_words(n, k)
    return mfma.contiguous().view(-1)[pw + n : pw + 2 * n]


def codes_from_fragment_major(q: torch.Tensor, m: int, k: int) -> torch.Tensor:
    """Fragment-major quantized activations (as written by the GPU quantizer) ->
    the reference's row-major int32 words [M, K/8] (``quantize_x``'s ``q``)."""
    flat = q.reshape(-1)
    return flip_activation_words(flat[fragment_word_index(m, k, q.device)])


def qcorr_from_fragment_major(q: torch.Tensor, m: int, k: int) -> torch.Tensor:
    """The qcorr words [M] stored after the fragment-major activation codes."""
    pw = ((m + 15) // 16) * 16 * ((k + 127) // 128) * 16
    return q.reshape(-1)[pw : pw + m]


# ---- E3M2 (OCP FP6: sign bit 5, exponent bits 4-2 with bias 3, mantissa bits 1-0) forms
# of the INT4 codes, read by the gfx950 FP6-MFMA gate/up GEMM.  A lane slot is six
# little-endian dwords holding 32 codes, code j in bits 6j .. 6j+5.
E3M2_MARKER_WORDS = 16


def e3m2_to_float(bits: torch.Tensor) -> torch.Tensor:
    """Values of 6-bit E3M2 patterns: (-1)^s 2^(e-3) (1 + m/4), subnormal (e = 0) m/16."""
    b = bits.to(torch.int64)
    e = (b >> 2) & 7
    man = (b & 3).to(torch.float64)
    mag = torch.where(e == 0, man / 16.0, torch.exp2((e - 3).to(torch.float64)) * (1.0 + man / 4.0))
    return torch.where((b >> 5) & 1 == 1, -mag, mag)


def _slot_codes(slot_bytes: torch.Tensor) -> torch.Tensor:
    """[..., 24] uint8 lane slots -> [..., 32] int8 codes.  Each slot is read as three
    little-endian 64-bit words; field j (bits 6j .. 6j+5) is decoded through the 64-entry
    value table of ``e3m2_to_float``.  Every field must be an integer value."""
    import numpy as np

    u = np.ascontiguousarray(slot_bytes.numpy()).view("<u8")  # [..., 3]
    words = [np.ascontiguousarray(u[..., i]) for i in range(3)]
    fields = []
    for j in range(32):
        w, off = divmod(6 * j, 64)
        f = words[w] >> np.uint64(off)
        if off > 58:
            f = f | (words[w + 1] << np.uint64(64 - off))
        fields.append((f & np.uint64(63)).astype(np.uint8))
    fields = np.stack(fields, axis=-1)
    vals = e3m2_to_float(torch.arange(64)).numpy()
    if not np.take((np.rint(vals) == vals).astype(np.uint8), fields).all():
        raise ValueError("E3M2 codes hold a non-integer value")
    return torch.from_numpy(np.take(np.rint(vals).astype(np.int8), fields))


def codes_from_e3m2_fragments(q6: torch.Tensor, m: int, k: int) -> torch.Tensor:
    """E3M2 activation fragments (``quantize_e3m2``'s q6, 1536 bytes per 16 rows x 128 k)
    -> int8 codes [M, K]."""
    mb, kb = (m + 15) // 16, (k + 127) // 128
    f = q6.reshape(-1)[: mb * kb * 1536].to(torch.uint8).reshape(mb, kb, 1536)
    slots = torch.cat((f[:, :, :1024].reshape(mb, kb, 64, 16), f[:, :, 1024:].reshape(mb, kb, 64, 8)), dim=-1)
    # [mb, kb, lane, 24] slots of row 16 mb + lane % 16, codes 128 kb + 32 (lane / 16) + j; only
    # the rows below M are decoded (the pad rows of the last block are never written)
    slots = slots.reshape(mb, kb, 4, 16, 24).permute(0, 3, 1, 2, 4).reshape(mb * 16, kb * 4, 24)[:m]
    return _slot_codes(slots).reshape(m, kb * 128)[:, :k]


def codes_from_e3m2_weight(w6: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """E3M2 column-pair weight int32 [N, 3K/16+16] -> (int8 codes [N, K], fp32 scales [N])."""
    n = int(w6.size(0))
    kb = (k + 127) // 128
    flat = w6.reshape(-1).contiguous()
    payload = flat[: n * kb * 24].view(torch.uint8).reshape(n // 32, kb, 3, 64, 16)
    rec = payload.permute(0, 1, 3, 2, 4).reshape(n // 32, kb, 64, 48)  # lane records
    slots = torch.stack((rec[..., :24], rec[..., 24:]), dim=2)  # [pair, kb, half, lane, 24]
    codes = _slot_codes(slots)  # column 32 p + 16 half + lane % 16, k 128 kb + 32 (lane / 16) + j
    codes = codes.reshape(n // 32, kb, 2, 4, 16, 32).permute(0, 2, 4, 1, 3, 5).reshape(n, kb * 128)
    scales = flat[n * kb * 24 : n * kb * 24 + n].view(torch.float32)
    return codes[:, :k], scales


def quant_activation_cpu(x: torch.Tensor, rotate: bool | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """CPU statement of the activation quant (pack.py:113-131): x [M, K] -> (codes [M, K], scale [M]).

    sdiv = amax/7 + 1e-12; codes = clamp(round_half_even(x'/sdiv), -7, 7);
    scale = sdiv * fp32(1/sqrt(K)) when rotating, else sdiv.
    """
    if x.dim() != 2:
        raise ValueError("quant_activation_cpu expects [M, K]")
    _, k = x.shape
    xf = x.detach().float()
    rot = should_rotate(k, rotate)
    if rot:
        xf = fwht_unnormalized(xf)
    sdiv = xf.abs().amax(dim=-1) / 7.0 + 1e-12
    scale = sdiv * (1.0 / math.sqrt(k)) if rot else sdiv
    codes = torch.round(xf / sdiv[:, None]).clamp(-7, 7).to(torch.int32)
    return codes, scale


def int4_gemm_ref(x: torch.Tensor, packed_w: torch.Tensor, rotate: bool | None = None) -> torch.Tensor:
    """CPU reference of one W4A4 linear (pack.py:134-145): fp32 matmul of the codes (exact,
    |acc| < 2^24), then (acc * s_a) * s_w rounded to fp16."""
    lead = x.shape[:-1]
    k = x.shape[-1]
    q_a, s_a = quant_activation_cpu(x.reshape(-1, k), rotate=rotate)
    q_w, s_w, k_w = unpack_linear_weight(packed_w)
    if k_w != k:
        raise ValueError(f"K mismatch act={k} weight={k_w}")
    acc = q_a.float() @ q_w.float().T
    y = acc * s_a[:, None] * s_w[None, :]
    return y.reshape(*lead, packed_w.shape[0]).to(torch.float16)


def layer_meta(name: str, packed: torch.Tensor, rotate: bool, has_bias: bool) -> dict[str, Any]:
    """Per-layer entry of meta.json (pack.py:148-157)."""
    n, row = packed.shape
    return {
        "name": name,
        "in_features": (row - 1) * 8,
        "out_features": n,
        "rotate": rotate,
        "has_bias": has_bias,
    }
