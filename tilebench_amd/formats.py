"""On-disk quantized weight formats -> the hip backend's layouts.

The W4A16 kernels take int4 weights as ``packed`` uint8 [K, N/2] (column n in
the low nibble of byte n/2 when n is even, the high nibble when odd), fp16
``scales`` [K/G, N] and ``zeros`` packed the same way [K/G, N/2], with groups
of G consecutive input channels.  The fp8 GEMM takes e4m3 (OCP, "fn") codes
of the weight transposed, WqT [N, K], with one fp32 scale per output column.

Checkpoints store these differently; the converters below (torch, any device,
run once at load time) restate the published conventions of the packers that
write them.  Those packers are not part of this repository or of the
reference (Tilebench has no quantized checkpoints); their conventions are:

* GPTQ (AutoGPTQ / GPTQModel, "gptq" v1 checkpoints): ``qweight`` int32
  [K/8, N], input channel 8i + j of column n in bits 4j..4j+3 of word [i, n];
  ``qzeros`` int32 [K/G, N/8], column 8i + j in bits 4j..4j+3 of word [g, i],
  storing zero - 1 (v1; "gptq_v2" stores the zero itself); ``scales`` fp16
  [K/G, N]; ``g_idx`` int32 [K], the group of each input channel.  With
  act-order (desc_act) the groups are not contiguous along K: the converter
  then returns the input-channel permutation that makes them contiguous, and
  the activations are permuted the same way (``permute_input``).
* AWQ (llm-awq / AutoAWQ GEMM layout): ``qweight`` int32 [K, N/8] and
  ``qzeros`` int32 [K/G, N/8], eight columns per word in the nibble order
  0, 2, 4, 6, 1, 3, 5, 7 (nibble j holds column 8i + AWQ_ORDER[j]); zeros are
  stored as is; ``scales`` fp16 [K/G, N].
* fp8 (e4m3) checkpoints: ``weight`` [N, K] (already K-contiguous, i.e. WqT),
  ``weight_scale`` per tensor (a scalar) or per output channel ([N] or
  [N, 1]); DeepSeek-V3-style checkpoints name it ``weight_scale_inv`` (the
  inverse of the quantisation factor, so again the dequantisation
  multiplier: W ~= Wq * weight_scale_inv).  MI300-era
  checkpoints use e4m3fnuz (exponent bias 8, NaN 0x80, max 240); those codes
  are re-encoded as e4m3fn by value: every fnuz value that is a multiple of
  2^-9 is an fn value, and the eight magnitudes that are odd multiples of
  2^-10 (all below 2^-6) round to nearest even.  Block
  scales (one per 128 x 128 tile, [ceil(N/128), ceil(K/128)]: DeepSeek-V3's
  weight_scale_inv) select the block-scaled GEMM (Fp8BlockWeights).
* Decode slab layout: not a checkpoint format but the W4A16 decode's own
  weight layout, converted once at load (w4a16_to_slabs below).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

#: AutoAWQ's nibble order: nibble j of a word holds column 8i + AWQ_ORDER[j].
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


@dataclass
class Int4Weights:
    """W4A16 operands in the hip layout, plus the input-channel permutation
    (None when the groups were already contiguous along K)."""
    packed: torch.Tensor   # uint8 [K, N/2]
    scales: torch.Tensor   # fp16 [K/G, N]
    zeros: torch.Tensor    # uint8 [K/G, N/2]
    group: int
    perm: torch.Tensor | None = None   # int64 [K]: row i of `packed` is input channel perm[i]


@dataclass
class Fp8Weights:
    """fp8 GEMM operands: e4m3fn codes of W^T and one fp32 scale per column."""
    wqT: torch.Tensor      # uint8 [N, K]
    sw: torch.Tensor       # fp32 [N]


@dataclass
class Fp8BlockWeights:
    """Block-scaled fp8 GEMM operands (tb_fp8_block_gemm): e4m3fn codes of W^T
    and one fp32 scale per 128 x 128 tile."""
    wqT: torch.Tensor      # uint8 [N, K]
    sw: torch.Tensor       # fp32 [ceil(N/128), K/128]
    block: int = 128


# ----------------------------------------------------------------------------- nibbles


def _nibbles_of_words(words: torch.Tensor) -> torch.Tensor:
    """int32 words [..., W] -> uint8 nibbles [..., W, 8], nibble j = bits 4j..4j+3."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(0, 32, 4, device=words.device, dtype=torch.int64)
    return ((w.unsqueeze(-1) >> shifts) & 0xF).to(torch.uint8)


def _words_of_nibbles(nib: torch.Tensor) -> torch.Tensor:
    """uint8 nibbles [..., W, 8] -> int32 words [..., W] (two's complement)."""
    shifts = torch.arange(0, 32, 4, device=nib.device, dtype=torch.int64)
    w = (nib.to(torch.int64) << shifts).sum(dim=-1)
    return torch.where(w >= 1 << 31, w - (1 << 32), w).to(torch.int32)


def pack_columns(codes: torch.Tensor) -> torch.Tensor:
    """uint8 codes [..., N] in [0, 15] -> uint8 [..., N/2], column n in the low
    nibble of byte n/2 for even n and in the high nibble for odd n."""
    if codes.shape[-1] % 2:
        raise ValueError("need an even number of columns")
    c = codes.to(torch.uint8)
    return c[..., 0::2] | (c[..., 1::2] << 4)


def unpack_columns(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_columns."""
    p = packed.to(torch.uint8)
    return torch.stack((p & 0xF, p >> 4), dim=-1).reshape(*p.shape[:-1], -1)


# ----------------------------------------------------------------------------- GPTQ


def gptq_codes(qweight: torch.Tensor) -> torch.Tensor:
    """GPTQ qweight int32 [K/8, N] -> uint8 codes [K, N] (K-packed, nibble j = row 8i + j)."""
    nib = _nibbles_of_words(qweight.transpose(0, 1))          # [N, K/8, 8]
    return nib.reshape(qweight.shape[1], -1).transpose(0, 1).contiguous()


def gptq_zero_codes(qzeros: torch.Tensor, zero_offset: int = 1) -> torch.Tensor:
    """GPTQ qzeros int32 [K/G, N/8] -> uint8 zero-points [K/G, N] (stored value
    + zero_offset: 1 for v1 checkpoints, 0 for v2), wrapped to 4 bits."""
    nib = _nibbles_of_words(qzeros).reshape(qzeros.shape[0], -1)
    return ((nib.to(torch.int16) + zero_offset) & 0xF).to(torch.uint8)


def gptq_to_tb(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, g_idx: torch.Tensor | None = None,
               zero_offset: int = 1) -> Int4Weights:
    """A GPTQ layer in the hip layout.  Without act-order (g_idx None or
    g_idx[k] == k // G) the rows keep their order; otherwise rows are sorted
    by group (stably), `perm` records the order, and each group must hold
    exactly G input channels."""
    q = gptq_codes(qweight)
    K, N = q.shape
    ngroups = scales.shape[0]
    if K % ngroups or tuple(scales.shape) != (ngroups, N) or tuple(qzeros.shape) != (ngroups, N // 8):
        raise ValueError(f"GPTQ shapes do not match: qweight {tuple(qweight.shape)}, qzeros {tuple(qzeros.shape)}, "
                         f"scales {tuple(scales.shape)}")
    G = K // ngroups
    z = gptq_zero_codes(qzeros, zero_offset)
    perm = None
    if g_idx is not None:
        g_idx = g_idx.to(torch.int64).reshape(-1)
        if g_idx.numel() != K or g_idx.min() < 0 or g_idx.max() >= ngroups:
            raise ValueError("g_idx must hold one group index in [0, K/G) per input channel")
        trivial = torch.arange(K, device=g_idx.device) // G
        if not torch.equal(g_idx, trivial):
            counts = torch.bincount(g_idx, minlength=ngroups)
            if not bool((counts == G).all()):
                raise ValueError("act-order g_idx must put exactly K/ngroups input channels in every group")
            perm = torch.sort(g_idx, stable=True).indices
            q = q[perm.to(q.device)]
    return Int4Weights(pack_columns(q), scales.to(torch.float16).contiguous(), pack_columns(z), G,
                       None if perm is None else perm.to(qweight.device))


def tb_to_gptq(w: Int4Weights, zero_offset: int = 1):
    """The inverse: (qweight, qzeros, scales, g_idx) of a GPTQ checkpoint."""
    q = unpack_columns(w.packed)
    K, N = q.shape
    G = w.group
    g_idx = torch.arange(K, device=q.device) // G
    if w.perm is not None:
        inv = torch.empty_like(w.perm)
        inv[w.perm] = torch.arange(K, device=w.perm.device)
        q = q[inv.to(q.device)]
        g_idx = g_idx[inv.to(q.device)]
    qweight = _words_of_nibbles(q.transpose(0, 1).reshape(N, K // 8, 8)).transpose(0, 1).contiguous()
    z = ((unpack_columns(w.zeros).to(torch.int16) - zero_offset) & 0xF).to(torch.uint8)
    qzeros = _words_of_nibbles(z.reshape(z.shape[0], N // 8, 8))
    return qweight, qzeros, w.scales, g_idx.to(torch.int32)


def permute_input(A: torch.Tensor, perm: torch.Tensor | None) -> torch.Tensor:
    """Activations in the converted weights' input-channel order (A[:, perm])."""
    return A if perm is None else A.index_select(-1, perm.to(A.device)).contiguous()


# ----------------------------------------------------------------------------- AWQ


def _awq_unpack(words: torch.Tensor) -> torch.Tensor:
    nib = _nibbles_of_words(words)                            # [R, N/8, 8], nibble j
    out = torch.empty_like(nib)
    out[..., list(AWQ_ORDER)] = nib                           # column AWQ_ORDER[j] <- nibble j
    return out.reshape(words.shape[0], -1)


def awq_to_tb(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> Int4Weights:
    """An AWQ (GEMM layout) layer in the hip layout."""
    q = _awq_unpack(qweight)
    K, N = q.shape
    ngroups = scales.shape[0]
    if K % ngroups or tuple(scales.shape) != (ngroups, N) or tuple(qzeros.shape) != (ngroups, N // 8):
        raise ValueError(f"AWQ shapes do not match: qweight {tuple(qweight.shape)}, qzeros {tuple(qzeros.shape)}, "
                         f"scales {tuple(scales.shape)}")
    z = _awq_unpack(qzeros)
    return Int4Weights(pack_columns(q), scales.to(torch.float16).contiguous(), pack_columns(z), K // ngroups)


def tb_to_awq(w: Int4Weights):
    """The inverse: (qweight, qzeros, scales) of an AWQ checkpoint."""
    if w.perm is not None:
        raise ValueError("AWQ has no input-channel permutation")

    def pack(codes):
        R, N = codes.shape
        c = codes.reshape(R, N // 8, 8)[..., list(AWQ_ORDER)]  # nibble j <- column AWQ_ORDER[j]
        return _words_of_nibbles(c)
    return pack(unpack_columns(w.packed)), pack(unpack_columns(w.zeros)), w.scales


# ----------------------------------------------------------------------------- decode slabs

SLAB_COLS = 64    # columns per slab
SLAB_UNIT = 32    # K rows per 1 KiB unit
_SLAB_SHIFT = (0, 16, 4, 20, 8, 24, 12, 28)   # bit of code i within its 32-bit word


def slab_shape(K: int, N: int) -> tuple[int, int, int]:
    """Shape of the slab layout of a [K, N] int4 matrix: uint8 [N/64, K/32, 1024]."""
    if K % SLAB_UNIT or N % SLAB_COLS or K <= 0 or N <= 0:
        raise ValueError(f"the slab layout needs K % {SLAB_UNIT} == 0 and N % {SLAB_COLS} == 0 (K={K} N={N})")
    return (N // SLAB_COLS, K // SLAB_UNIT, 1024)


def w4a16_to_slabs(packed: torch.Tensor) -> torch.Tensor:
    """Packed int4 weights uint8 [K, N/2] -> the decode's slab layout, uint8
    [N/64, K/32, 1024], a weight format of its own (converted once, at load).

    Slab s holds columns 64 s .. 64 s + 63 as K/32 units of 1 KiB.  In unit u,
    lane l's 16 bytes are four little-endian 32-bit words; word b holds the
    codes of column 64 s + 16 b + l % 16 at rows 32 u + 8 (l / 16) + i,
    i = 0..7, code i at bit (i % 2) * 16 + (i / 2) * 4.  On a GPU tensor the
    library's tb_w4a16_repack_slabs writes it (one launch); on a CPU tensor the
    same map is evaluated with torch indexing."""
    if packed.dtype != torch.uint8 or packed.dim() != 2:
        raise TypeError("w4a16_to_slabs expects packed uint8 [K, N/2] weights")
    K, N = packed.shape[0], packed.shape[1] * 2
    shape = slab_shape(K, N)
    packed = packed.contiguous()
    if packed.is_cuda:
        from tilebench_amd import runtime as rt

        rt.require_device()
        out = torch.empty(shape, dtype=torch.uint8, device=packed.device)
        rt.call("tb_w4a16_repack_slabs", packed.data_ptr(), out.data_ptr(), K, N, rt.stream_handle(packed.device))
        return out
    # codes q[k, n] with k = 32 u + 8 r + i and n = 64 s + 16 b + c, viewed as [u, r, i, s, b, c]
    q = unpack_columns(packed).to(torch.int32).reshape(K // 32, 4, 8, N // 64, 4, 16)
    shifts = torch.tensor(_SLAB_SHIFT, dtype=torch.int32).reshape(1, 1, 1, 1, 1, 8)
    q = q.permute(3, 0, 1, 5, 4, 2)                  # [s, u, r, c, b, i]: lane l = 16 r + c
    words = (q << shifts).sum(dim=-1, dtype=torch.int32)
    return words.contiguous().view(torch.uint8).reshape(shape)


def w4a16_from_slabs(slabs: torch.Tensor) -> torch.Tensor:
    """The inverse of w4a16_to_slabs: uint8 [N/64, K/32, 1024] -> packed
    uint8 [K, N/2] (torch indexing, any device)."""
    if slabs.dtype != torch.uint8 or slabs.dim() != 3 or slabs.shape[2] != 1024:
        raise TypeError("w4a16_from_slabs expects uint8 [N/64, K/32, 1024] slabs")
    S, U = slabs.shape[0], slabs.shape[1]
    words = slabs.contiguous().view(torch.int32).reshape(S, U, 4, 16, 4, 1)   # [s, u, r, c, b, 1]
    shifts = torch.tensor(_SLAB_SHIFT, dtype=torch.int32, device=slabs.device)
    q = (words >> shifts) & 15                        # [s, u, r, c, b, i]
    q = q.permute(1, 2, 5, 0, 4, 3).reshape(U * 32, S * 64)   # [u, r, i, s, b, c]
    return pack_columns(q.to(torch.uint8))


# ----------------------------------------------------------------------------- fp8


def _fnuz_to_fn_codes(codes: torch.Tensor) -> torch.Tensor:
    """e4m3fnuz codes -> e4m3fn codes of the same values: decoded exactly to
    fp32, then encoded round-to-nearest-even (exact except the odd multiples
    of 2^-10, below fn's finest step 2^-9); NaN stays NaN."""
    return codes.view(torch.float8_e4m3fnuz).to(torch.float32).to(torch.float8_e4m3fn).view(torch.uint8)


def fp8_checkpoint_to_tb(weight: torch.Tensor, weight_scale: torch.Tensor | float | None = None, *,
                         weight_scale_inv: torch.Tensor | float | None = None) -> Fp8Weights | Fp8BlockWeights:
    """An fp8 linear layer (weight [N, K] in e4m3fn or e4m3fnuz, or its uint8
    codes as e4m3fn) -> the operands of the GEMM its scale layout needs:
    a per-tensor or per-output-channel scale gives Fp8Weights (WqT codes
    [N, K], sw fp32 [N]) for tb_fp8_scaled_gemm; a scale per 128 x 128 tile
    ([ceil(N/128), ceil(K/128)], DeepSeek-V3's weight_scale_inv) gives
    Fp8BlockWeights for tb_fp8_block_gemm (K must then be a multiple of 128).

    Both checkpoint keys hold the dequantisation multiplier, W ~= Wq * scale:
    `weight_scale` (compressed-tensors / vLLM fp8 layers) and
    `weight_scale_inv` (DeepSeek-V3 and transformers' FineGrainedFP8, where the
    name says it is the inverse of the quantisation factor 448 / amax, i.e.
    amax / 448).  Either one is therefore sw as it stands."""
    if (weight_scale is None) == (weight_scale_inv is None):
        raise ValueError("give exactly one of weight_scale and weight_scale_inv")
    N, K = weight.shape
    if weight.dtype == torch.float8_e4m3fn or weight.dtype == torch.uint8:
        codes = weight.view(torch.uint8) if weight.dtype != torch.uint8 else weight
    elif weight.dtype == torch.float8_e4m3fnuz:
        codes = _fnuz_to_fn_codes(weight.view(torch.uint8))
    else:
        raise TypeError(f"unsupported fp8 weight dtype {weight.dtype}")
    s = weight_scale if weight_scale is not None else weight_scale_inv
    s = torch.as_tensor(s, dtype=torch.float32, device=weight.device)
    blocks = (-(-N // 128), -(-K // 128))
    if s.dim() == 2 and tuple(s.shape) == blocks and tuple(s.shape) != (N, 1):
        if K % 128:
            raise ValueError(f"block-scaled fp8 weight [{N}, {K}]: the block GEMM needs K % 128 == 0")
        return Fp8BlockWeights(codes.contiguous(), s.contiguous())
    if s.numel() == 1:
        s = s.reshape(1).expand(N)
    elif s.numel() == N and (s.dim() == 1 or (s.dim() == 2 and s.shape[1] == 1)):
        s = s.reshape(N)
    else:
        raise ValueError(f"fp8 scale of shape {tuple(s.shape)} for a [{N}, {K}] weight: expected a scalar, [N], "
                         f"[N, 1] or 128 x 128 blocks {blocks}")
    return Fp8Weights(codes.contiguous(), s.contiguous().to(torch.float32))


# ----------------------------------------------------------------------------- files


def load_safetensors_layer(path, prefix: str, fmt: str, device="cpu", zero_offset: int = 1):
    """Read one quantized linear layer from a local safetensors file.

    fmt "gptq": `{prefix}.qweight/.qzeros/.scales[/.g_idx]`; "awq": the same
    without g_idx; "fp8": `{prefix}.weight` and `.weight_scale` (or
    `.weight_scale_inv`).  Only local files; nothing is fetched."""
    from safetensors import safe_open

    with safe_open(str(path), framework="pt", device=str(device)) as f:
        keys = set(f.keys())

        def get(name, required=True):
            key = f"{prefix}.{name}"
            if key not in keys:
                if required:
                    raise KeyError(f"{key} not in {path}")
                return None
            return f.get_tensor(key)

        if fmt == "gptq":
            return gptq_to_tb(get("qweight"), get("qzeros"), get("scales"), get("g_idx", False), zero_offset)
        if fmt == "awq":
            return awq_to_tb(get("qweight"), get("qzeros"), get("scales"))
        if fmt == "fp8":
            return fp8_checkpoint_to_tb(get("weight"), get("weight_scale", False),
                                        weight_scale_inv=get("weight_scale_inv", False))
    raise ValueError(f"unknown format {fmt!r} (gptq, awq, fp8)")
