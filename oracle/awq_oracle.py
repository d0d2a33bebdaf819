"""CPU oracle for the AWQ W4A16 linear path (test infrastructure, never product).

This module restates, in numpy and CPU torch, the arithmetic of SGLite's AWQ
linear path so that the HIP engine can be checked against it.  Only the test
suite, the package smoke check and the benchmark's CPU-baseline leg import it;
the product path never does.

Reference functions restated here (paths relative to
``python/sglite/srt/model_executor/``):

* nibble order      -- layers/quantization/awq_triton.py:53-62 (reverse order
                       [0,4,1,5,2,6,3,7] and shifts = 4*order) and
                       layers/quantization/marlin_utils.py:249-282, 340-347
                       (unpack_cols + argsort([0,2,4,6,1,3,5,7])).
* dequantisation    -- layers/quantization/awq_triton.py:99-101, 119-122:
                       W = ((q >> s) & 0xF  -  (z >> s) & 0xF) * scale, with the
                       group row = k // group_size, one rounding to the output
                       dtype.
* GEMM              -- layers/quantization/awq.py:133-147 and
                       awq_triton.py:144-195: y = x @ W, then ``+ bias`` in the
                       activation dtype.  The contract accumulates in fp32 (the
                       Marlin path's ``use_fp32_reduce=True``,
                       marlin_utils.py:16, 408), not the Triton fallback's fp16.
* gated MLP block   -- models/blocks.py:51-57: gate_up_proj (the merged
                       projection, gate columns first), silu_and_mul /
                       gelu_and_mul (layers/activation.py:11-23) on the rounded
                       GEMM output, rounded once, then down_proj.
* fused MoE         -- layers/fused_moe/fused.py:11-31 (softmax top-k and
                       renormalisation), fused.py:101-202 (GEMM1, silu_and_mul
                       with the gate half first, GEMM2 times the routed weight
                       in fp32, sum over top-k), kernels/triton/fused_moe.py:
                       7-50 and 174-178.

How each part is pinned (tests/test_oracle.py):
  unpack/pack         KAT words (0x76543210 -> [0,4,1,5,2,6,3,7],
                      [0..7] -> 0x75316420), a literal simulation of the
                      Triton kernel's triple ``interleave`` + shifts, and a
                      literal restatement of the Marlin unpack + argsort path.
  dequantize          exhaustive (q, z) x scale sweep against numpy's float16
                      rounding of the float64 product (fp16) and a bit-level
                      round-to-nearest-even (bf16); q == z gives 0; z=0, s=1
                      gives q; s = 2^-g pins the group mapping.
  awq_gemm            float64 brute force on tiny shapes; exact integer
                      products with s=1, z=0; one-hot rows give rows of W.
  repack/unrepack     round trip on random and ragged shapes; the repacked
                      dequantisation equals ``dequantize``.
  gated_mlp_awq       in fp32 activations (no rounding between the steps)
                      against the dense GatedMLP layer of the package run on
                      the dequantized weights, and at fp16 against the steps
                      composed by hand with a swapped gate/up order failing.
  MoE                 explicit per-(token, slot) loops against the vectorised
                      form; softmax/top-k are torch's textbook routines.
The reference's own tests are not shipped (its .gitignore lists ``tests``), so
no reference golden vectors exist for this path.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np
import torch

# Nibble p of a packed int32 holds logical column 8j + AWQ_ORDER[p]
# (marlin_utils.py:340-347 undoes exactly this interleave).
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
# Logical column 8j + i lives in nibble REVERSE_AWQ_ORDER[i]
# (awq_triton.py:53-62: reverse order [0,4,1,5,2,6,3,7], shift = 4 * order).
REVERSE_AWQ_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)

_DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def _as_u32(a) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        a = a.cpu().numpy()
    return np.ascontiguousarray(a).astype(np.int64).astype(np.uint32)


def unpack_awq(packed) -> np.ndarray:
    """Unpack AWQ int32 words [R, C/8] into logical 4-bit values [R, C] (int32).

    q[r, 8j+i] = (packed[r, j] >> 4*REVERSE_AWQ_ORDER[i]) & 0xF
    (awq_triton.py:53-62, 119-120; the shift is logical here, which equals the
    reference's arithmetic shift after the & 0xF mask).
    """
    p = _as_u32(packed)
    R, C8 = p.shape
    out = np.empty((R, C8, 8), dtype=np.int32)
    for i in range(8):
        out[:, :, i] = ((p >> np.uint32(4 * REVERSE_AWQ_ORDER[i])) & np.uint32(0xF)).astype(np.int32)
    return out.reshape(R, C8 * 8)


def pack_awq(q) -> np.ndarray:
    """Pack logical 4-bit values [R, C] into AWQ int32 words [R, C/8].

    Inverse of :func:`unpack_awq`: nibble p receives column 8j + AWQ_ORDER[p].
    """
    if isinstance(q, torch.Tensor):
        q = q.cpu().numpy()
    q = np.asarray(q).astype(np.uint32)
    R, C = q.shape
    if C % 8:
        raise ValueError("column count must be a multiple of 8")
    q = q.reshape(R, C // 8, 8)
    w = np.zeros((R, C // 8), dtype=np.uint32)
    for p in range(8):
        w |= (q[:, :, AWQ_ORDER[p]] & np.uint32(0xF)) << np.uint32(4 * p)
    return w.view(np.int32)


def resolve_group_size(group_size: int, K: int) -> int:
    """Group size -1 means one group over all of K (awq_marlin.py:182-184)."""
    return K if group_size == -1 else group_size


def dequantize(qweight, qzeros, scales: torch.Tensor, group_size: Optional[int] = None) -> torch.Tensor:
    """Dequantise AWQ tensors to W[K, N] in ``scales.dtype``.

    W[k, n] = rnd((q[k, n] - z[k // G, n]) * s[k // G, n])   (awq_triton.py:119-122)

    q - z is an exact integer in [-15, 15]; its product with an fp16 or bf16
    scale is exact in float64, so rounding the float64 product once to the
    output dtype is the single round-to-nearest-even of the reference.
    ``group_size`` defaults to K // qzeros.shape[0] (awq_triton.py:155-157).
    """
    q = unpack_awq(qweight)
    z = unpack_awq(qzeros)
    K, N = q.shape
    if group_size is None:
        group_size = K // z.shape[0]
    G = resolve_group_size(group_size, K)
    g_of_k = np.arange(K) // G
    s = scales.detach().cpu().to(torch.float64).numpy()
    diff = (q - z[g_of_k, :]).astype(np.float64)
    w64 = diff * s[g_of_k, :]
    return torch.from_numpy(w64).to(scales.dtype)


def dequantize_torch(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                     group_size: Optional[int] = None) -> torch.Tensor:
    """:func:`dequantize` in multithreaded CPU torch (the CPU baseline's dequantisation).

    Same arithmetic: the nibble of logical column 8j + i is
    (word >> 4 * REVERSE_AWQ_ORDER[i]) & 0xF, q - z is an exact integer, and
    its product with the scale is exact in fp32 (a 4-bit by an 11- or 8-bit
    significand), so converting the fp32 product is the one rounding.  Pinned
    bit for bit against :func:`dequantize` in tests/test_oracle.py.
    """
    K, N8 = qweight.shape
    N = N8 * 8
    if group_size is None:
        group_size = K // qzeros.shape[0]
    G = resolve_group_size(group_size, K)
    shifts = torch.tensor([4 * o for o in REVERSE_AWQ_ORDER], dtype=torch.int32)

    def unpack(p: torch.Tensor) -> torch.Tensor:
        return ((p.unsqueeze(-1) >> shifts) & 0xF).reshape(p.shape[0], N)

    q = unpack(qweight.cpu()).to(torch.float32)
    z = unpack(qzeros.cpu()).to(torch.float32)
    s = scales.cpu().to(torch.float32)
    q = q.view(K // G, G, N)
    q.sub_(z.unsqueeze(1)).mul_(s.unsqueeze(1))
    return q.view(K, N).to(scales.dtype)


def awq_gemm(x: torch.Tensor, qweight, qzeros, scales: torch.Tensor, bias: Optional[torch.Tensor] = None,
             group_size: Optional[int] = None) -> torch.Tensor:
    """fp32-accumulated AWQ linear: y = rnd(x @ W) (+ bias in the activation dtype).

    Mirrors awq.py:133-147 (reshape to [M, K], GEMM, ``out + bias``, reshape to
    x.shape[:-1] + (N,)) with the accumulation done in fp32 as in the Marlin
    path (marlin_utils.py:408).
    """
    W = dequantize(qweight, qzeros, scales, group_size)
    K, N = W.shape
    x2 = x.detach().cpu().reshape(-1, K)
    y = (x2.float() @ W.float()).to(x.dtype)
    if bias is not None:
        y = y + bias.detach().cpu().to(y.dtype)
    return y.reshape(*x.shape[:-1], N)


def awq_gemm_f64(x: torch.Tensor, qweight, qzeros, scales: torch.Tensor, group_size: Optional[int] = None) -> np.ndarray:
    """Brute-force float64 product x @ W with W from :func:`dequantize` (tiny shapes only)."""
    W = dequantize(qweight, qzeros, scales, group_size).to(torch.float64).numpy()
    xs = x.detach().cpu().to(torch.float64).numpy().reshape(-1, W.shape[0])
    M, K = xs.shape
    N = W.shape[1]
    out = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for k in range(K):
            if xs[m, k] != 0.0:
                out[m] += xs[m, k] * W[k]
    return out


# ---------------------------------------------------------------------------
# CDNA4 tile layout (the engine's own repacked format; specified here so the
# device repack can be checked bit for bit).
#
# Weights: tiles of 16 output columns x 128 input rows, 1 KiB each, tile
# (nt, kt) at byte offset (nt * KT + kt) * 1024 with KT = ceil(K / 128).
# Inside a tile, lane l (0..63) owns 16 bytes = 4 little-endian uint32 words;
# word w holds column n = 16*nt + l % 16 and rows k0 .. k0+7 with
# k0 = 128*kt + 32*w + 8*(l // 16); nibble p holds row k0 + AWQ_ORDER[p].
# Out-of-range rows/columns hold 0.
#
# Scales: [NT][NG][16] in the scale dtype, NG = K // G (0 for padded columns).
# Zeros:  [NT][NG] uint64, nibble c = zero point of column 16*nt + c.
# The zeros array starts right after the scales array in one buffer.
# ---------------------------------------------------------------------------

TILE_N = 16
TILE_K = 128


def repacked_shapes(K: int, N: int, G: int) -> Dict[str, int]:
    NT = -(-N // TILE_N)
    KT = -(-K // TILE_K)
    NG = K // G
    return {"NT": NT, "KT": KT, "NG": NG,
            "w_bytes": NT * KT * 1024,
            "s_bytes": NT * NG * 16 * 2,
            "z_bytes": NT * NG * 8}


def repack_cdna4(qweight, qzeros, scales: torch.Tensor, group_size: int) -> Tuple[np.ndarray, np.ndarray]:
    """Return (weights uint8[w_bytes], scale_zero uint8[s_bytes + z_bytes])."""
    q = unpack_awq(qweight)
    z = unpack_awq(qzeros)
    K, N = q.shape
    G = resolve_group_size(group_size, K)
    sh = repacked_shapes(K, N, G)
    NT, KT, NG = sh["NT"], sh["KT"], sh["NG"]
    qp = np.zeros((KT * TILE_K, NT * TILE_N), dtype=np.uint32)
    qp[:K, :N] = q
    # qp[kt, w, lg, j, nt, c] with k = 128 kt + 32 w + 8 lg + j, n = 16 nt + c
    v = qp.reshape(KT, 4, 4, 8, NT, 16)
    words = np.zeros((NT, KT, 4, 16, 4), dtype=np.uint32)  # [nt, kt, lg, c, w]
    for p in range(8):
        j = AWQ_ORDER[p]
        # v[kt, w, lg, j, nt, c] at fixed j -> [nt, kt, lg, c, w]
        words |= v[:, :, :, j, :, :].transpose(3, 0, 2, 4, 1) << np.uint32(4 * p)
    wbuf = words.reshape(-1).view(np.uint8).copy()
    assert wbuf.size == sh["w_bytes"]

    s = scales.detach().cpu()
    sp = torch.zeros((NG, NT * TILE_N), dtype=s.dtype)
    sp[:, :N] = s
    s_r = sp.reshape(NG, NT, 16).permute(1, 0, 2).contiguous()
    sbytes = s_r.view(torch.int16).numpy().view(np.uint8).reshape(-1)
    zp = np.zeros((NG, NT * TILE_N), dtype=np.uint64)
    zp[:, :N] = z
    zr = zp.reshape(NG, NT, 16).transpose(1, 0, 2)
    zw = np.zeros((NT, NG), dtype=np.uint64)
    for c in range(16):
        zw |= zr[:, :, c] << np.uint64(4 * c)
    zbytes = zw.reshape(-1).view(np.uint8)
    return wbuf, np.concatenate([sbytes, zbytes])


def unrepack_cdna4(wbuf: np.ndarray, szbuf: np.ndarray, K: int, N: int, group_size: int,
                   dtype: torch.dtype) -> Tuple[np.ndarray, np.ndarray, torch.Tensor]:
    """Inverse of :func:`repack_cdna4` (returns AWQ qweight, qzeros, scales)."""
    G = resolve_group_size(group_size, K)
    sh = repacked_shapes(K, N, G)
    NT, KT, NG = sh["NT"], sh["KT"], sh["NG"]
    words = np.ascontiguousarray(wbuf).view(np.uint32).reshape(NT, KT, 4, 16, 4)
    v = np.zeros((KT, 4, 4, 8, NT, 16), dtype=np.uint32)
    for p in range(8):
        v[:, :, :, AWQ_ORDER[p], :, :] = ((words >> np.uint32(4 * p)) & np.uint32(0xF)).transpose(1, 4, 2, 0, 3)
    q = v.reshape(KT * TILE_K, NT * TILE_N)[:K, :N]
    sb = np.ascontiguousarray(szbuf[: sh["s_bytes"]]).view(np.int16)
    s_r = torch.from_numpy(sb.copy()).view(dtype).reshape(NT, NG, 16)
    scales = s_r.permute(1, 0, 2).reshape(NG, NT * TILE_N)[:, :N].contiguous()
    zw = np.ascontiguousarray(szbuf[sh["s_bytes"]: sh["s_bytes"] + sh["z_bytes"]]).view(np.uint64).reshape(NT, NG)
    z = np.zeros((NG, NT * 16), dtype=np.int32)
    for c in range(16):
        z[:, c::16] = ((zw >> np.uint64(4 * c)) & np.uint64(0xF)).astype(np.int32).T
    return pack_awq(q), pack_awq(z[:, :N]), scales


# ---------------------------------------------------------------------------
# Fused MoE (config: experts stacked on dim 0, AWQ gate_up [E, H, 2I] and
# down [E, I, H] in the AWQ orientation of a linear, i.e. qweight [E, K, N/8]).
# ---------------------------------------------------------------------------

def fused_topk(router_logits: torch.Tensor, topk: int, renormalize: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """softmax(fp32 logits) -> top-k -> optional renormalise (fused.py:11-31)."""
    p = torch.softmax(router_logits.detach().cpu().float(), dim=-1)
    w, ids = torch.topk(p, topk, dim=-1)
    if renormalize:
        w = w / (w.sum(dim=-1, keepdim=True) + 1e-8)
    return w, ids.to(torch.int32)


def silu_and_mul(h: torch.Tensor) -> torch.Tensor:
    """silu(h[..., :d]) * h[..., d:] in fp32 (activation.py:11-15: gate half first)."""
    d = h.shape[-1] // 2
    hf = h.float()
    return torch.nn.functional.silu(hf[..., :d]) * hf[..., d:]


def gelu_and_mul(h: torch.Tensor) -> torch.Tensor:
    """gelu(h[..., :d]) * h[..., d:] in fp32 with the erf form of GELU (activation.py:18-23)."""
    d = h.shape[-1] // 2
    hf = h.float()
    return torch.nn.functional.gelu(hf[..., :d]) * hf[..., d:]


_ACT = {"silu": silu_and_mul, "gelu": gelu_and_mul}


def gated_mlp_dequantized(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor,
                          activation: str = "silu") -> torch.Tensor:
    """GatedMLP.forward (blocks.py:51-57) on dequantized weights ([H, 2I] gate columns first, [I, H]):
    y = rnd(x @ W_gate_up) in fp32, h = rnd(act(gate) * up), out = rnd(h @ W_down)."""
    dt = x.dtype
    y = (x.detach().cpu().float() @ w_gate_up.float()).to(dt)
    h = _ACT[activation](y).to(dt)
    return (h.float() @ w_down.float()).to(dt)


def gated_mlp_awq(x: torch.Tensor, gate_up: Dict[str, torch.Tensor], down: Dict[str, torch.Tensor],
                  group_size: int, activation: str = "silu") -> torch.Tensor:
    """GatedMLP.forward on AWQ weights: :func:`gated_mlp_dequantized` of the :func:`dequantize`
    weights, so each GEMM is exactly :func:`awq_gemm` (no bias)."""
    wgu = dequantize(gate_up["qweight"], gate_up["qzeros"], gate_up["scales"], group_size)
    wdn = dequantize(down["qweight"], down["qzeros"], down["scales"], group_size)
    return gated_mlp_dequantized(x, wgu, wdn, activation)


def moe_align_block_size(topk_ids, block_size: int, num_experts: int):
    """Stable counting sort of the routed rows by expert (fused.py:34-61).

    Returns ``(sorted_ids, expert_ids, num_tokens_post_pad, offsets)`` as numpy
    int32 arrays: expert e's rows occupy ``sorted_ids[offsets[e]:offsets[e+1]]``
    in increasing row order, padded to a multiple of ``block_size`` with the
    sentinel ``n = topk_ids.size``; ``expert_ids[b]`` is the expert of block b
    (-1 past the last block).  Ids outside ``[0, num_experts)`` are dropped.
    The sgl_kernel layout is not observable through the MoE output (rows are
    independent), so its bucket order is this build's choice: stable."""
    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    n = ids.size
    cap = n + num_experts * (block_size - 1)
    bcap = (cap + block_size - 1) // block_size
    sorted_ids = np.full(cap, -7, dtype=np.int32)  # -7: never written (not read by consumers)
    expert_ids = np.full(bcap, -1, dtype=np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    pos = 0
    for e in range(num_experts):
        rows = np.nonzero(ids == e)[0]
        offsets[e] = pos
        sorted_ids[pos:pos + rows.size] = rows
        padded = -(-rows.size // block_size) * block_size
        sorted_ids[pos + rows.size:pos + padded] = n
        expert_ids[pos // block_size:(pos + padded) // block_size] = e
        pos += padded
    offsets[num_experts] = pos
    return sorted_ids, expert_ids, np.array([pos], dtype=np.int32), offsets


def moe_grouped_gemm(a: torch.Tensor, w: Dict[str, torch.Tensor], topk_weights: Optional[torch.Tensor],
                     topk_ids: torch.Tensor, top_k: int, group_size: int, activation: Optional[str] = None,
                     mul_routed_weight: bool = False) -> torch.Tensor:
    """One grouped GEMM of the MoE path per routed row r = t * topk + j
    (triton/fused_moe.py:54-183): ``a[r // top_k] @ W[expert(r)]`` in fp32,
    times ``topk_weights[r]`` when ``mul_routed_weight``, cast to a's dtype;
    with an ``activation`` the cast output's gate/up halves are combined as
    act(gate) * up in fp32 and cast again (activation.py:11-23).
    ``w`` holds expert-stacked ``qweight``/``qzeros``/``scales``."""
    dt = a.dtype
    ids = topk_ids.reshape(-1).cpu().long()
    n = ids.numel()
    af = a.detach().cpu().float()
    tw = None if topk_weights is None else topk_weights.reshape(-1).cpu().float()
    N = w["qweight"].shape[2] * 8
    out = torch.zeros((n, N // 2 if activation else N), dtype=dt)
    for e in torch.unique(ids).tolist():
        if e < 0 or e >= w["qweight"].shape[0]:
            continue
        rows = torch.nonzero(ids == e, as_tuple=True)[0]
        W = dequantize(w["qweight"][e], w["qzeros"][e], w["scales"][e], group_size).float()
        y = af[rows // top_k] @ W
        if mul_routed_weight:
            y = y * tw[rows][:, None]
        y = y.to(dt)
        if activation:
            y = _ACT[activation](y).to(dt)
        out[rows] = y
    return out


def fused_moe_awq(x: torch.Tensor, w1: Dict[str, torch.Tensor], w2: Dict[str, torch.Tensor],
                  topk_weights: torch.Tensor, topk_ids: torch.Tensor, group_size: int, activation: str = "silu",
                  apply_router_weight_on_input: bool = False, group_size2: Optional[int] = None) -> torch.Tensor:
    """Grouped AWQ MoE following fused.py:101-202 and triton/fused_moe.py:7-50, 174-178.

    GEMM1 per (token, slot) in fp32 (times the routed weight when it is
    applied on the input), cast to the activation dtype; act_and_mul
    (computed in fp32, cast); GEMM2 in fp32 times the routed weight (fp32)
    before the cast otherwise; the top-k outputs are summed in fp32 and cast.
    ``w1``/``w2`` hold expert-stacked ``qweight``/``qzeros``/``scales``.
    """
    dt = x.dtype
    T, H = x.shape
    k = topk_ids.shape[1]
    g2 = group_size if group_size2 is None else group_size2
    h2 = moe_grouped_gemm(x, w1, topk_weights, topk_ids, k, group_size, activation, apply_router_weight_on_input)
    y = moe_grouped_gemm(h2, w2, topk_weights, topk_ids, 1, g2, None, not apply_router_weight_on_input)
    return moe_sum_reduce(y.view(T, k, -1))


def moe_sum_reduce(y: torch.Tensor) -> torch.Tensor:
    """out[t] = rnd(sum_j y[t, j]) with an fp32 sum (triton/fused_moe.py:7-50)."""
    return y.float().sum(dim=1).to(y.dtype)


def fused_moe_awq_loops(x, w1, w2, topk_weights, topk_ids, group_size) -> torch.Tensor:
    """Explicit per-(token, slot) loop form of :func:`fused_moe_awq` (silu, tiny shapes only)."""
    dt = x.dtype
    T, H = x.shape
    k = topk_ids.shape[1]
    out = []
    for t in range(T):
        acc = None
        for j in range(k):
            e = int(topk_ids[t, j])
            W1 = dequantize(w1["qweight"][e], w1["qzeros"][e], w1["scales"][e], group_size).float()
            W2 = dequantize(w2["qweight"][e], w2["qzeros"][e], w2["scales"][e], group_size).float()
            h1 = (x[t].float() @ W1).to(dt)
            d = h1.shape[0] // 2
            g = h1[:d].float()
            h2 = (g / (1.0 + torch.exp(-g)) * h1[d:].float()).to(dt)
            y = ((h2.float() @ W2) * float(topk_weights[t, j])).to(dt).float()
            acc = y if acc is None else acc + y
        out.append(acc)
    return torch.stack(out).to(dt)


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (weights/scales/activations as the workloads state).
# ---------------------------------------------------------------------------

def make_awq_linear(K: int, N: int, group_size: int = 128, seed: int = 0,
                    dtype: torch.dtype = torch.float16) -> Dict[str, torch.Tensor]:
    """Nibbles uniform 0..15, scales uniform [0.002, 0.02], drawn in this order:
    q [K, N], z [K/G, N], s [K/G, N] from one torch.Generator seeded with ``seed``."""
    G = resolve_group_size(group_size, K)
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)
    z = torch.randint(0, 16, (K // G, N), generator=g, dtype=torch.int32)
    s = (torch.rand((K // G, N), generator=g) * 0.018 + 0.002).to(dtype)
    return {"qweight": torch.from_numpy(pack_awq(q)), "qzeros": torch.from_numpy(pack_awq(z)), "scales": s}


def make_activation(M: int, K: int, seed: int, dtype: torch.dtype = torch.float16) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn((M, K), generator=g).to(dtype)


ADVERSARIAL_KINDS = ("mean10", "outliers", "near_max")


def make_adversarial_activation(M: int, K: int, kind: str, seed: int,
                                dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Activations that stress the fp32 accumulation of the decode kernels:

    * ``mean10``: N(10, 1), a large common mean (sum_k x grows like 10 K);
    * ``outliers``: N(0, 1) with 1% of the channels scaled by 300 and two
      channels at +-1000 (the outlier channels AWQ's scales are chosen for);
    * ``near_max``: N(0, 1) with two channels at +-5e4 (fp16 near its maximum;
      with |W| <= 0.3 the outputs stay finite).
    The outlier channels are the same for every row."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g)
    ch = torch.randperm(K, generator=g)
    if kind == "mean10":
        x = x + 10.0
    elif kind == "outliers":
        x[:, ch[:max(1, K // 100)]] *= 300.0
        x[:, ch[K // 100]] = 1000.0
        x[:, ch[K // 100 + 1]] = -1000.0
    elif kind == "near_max":
        x[:, ch[0]] = 5.0e4
        x[:, ch[1]] = -5.0e4
    else:
        raise ValueError(f"unknown activation kind {kind!r}")
    return x.to(dtype)


def elementwise_ok(out: torch.Tensor, ref: torch.Tensor, rtol: float, atol_frac: float) -> Tuple[bool, float]:
    """|out - ref| <= rtol * |ref| + atol_frac * max|ref| for every element; also the worst ratio of
    the error to that bound (<= 1 passes)."""
    o = out.detach().cpu().float()
    r = ref.detach().cpu().float()
    bound = rtol * r.abs() + atol_frac * float(r.abs().max())
    ratio = float(((o - r).abs() / bound.clamp_min(1e-30)).max()) if o.numel() else 0.0
    return bool(torch.isfinite(o).all()) and ratio <= 1.0, ratio


def tolerance_ok(out: torch.Tensor, ref: torch.Tensor, rel: float = 2e-2) -> Tuple[bool, float, float]:
    """The GEMM contract: max|out - ref| <= rel * max|ref|."""
    o = out.detach().cpu().float()
    r = ref.detach().cpu().float()
    err = float((o - r).abs().max()) if o.numel() else 0.0
    mx = float(r.abs().max()) if r.numel() else 0.0
    return err <= rel * mx or (mx == 0.0 and err == 0.0), err, mx


def bf16_round_bits(x64: np.ndarray) -> np.ndarray:
    """Round float64 values (exactly representable in fp32) to bf16 bit patterns
    by integer round-to-nearest-even on the fp32 encoding (independent of torch)."""
    f = x64.astype(np.float32).view(np.uint32).astype(np.uint64)
    lsb = (f >> np.uint64(16)) & np.uint64(1)
    r = (f + np.uint64(0x7FFF) + lsb) >> np.uint64(16)
    return r.astype(np.uint16)


def gemm_bytes(M: int, N: int, K: int, G: int = 128, act_bytes: int = 2) -> int:
    """Algorithmic HBM bytes of one linear: int4 weights, packed zeros, scales, x, y."""
    return K * N // 2 + (K // G) * N // 2 + (K // G) * N * 2 + act_bytes * M * K + act_bytes * M * N


def gemm_flops(M: int, N: int, K: int) -> int:
    return 2 * M * N * K


__all__ = [name for name in dir() if not name.startswith("_") and name not in ("annotations", "math", "np", "torch")]
