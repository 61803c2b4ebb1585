"""Synthetic layers generated on the GPU, for benchmarks at full model sizes.

Expert weights are drawn N(0, std) per (layer, expert, projection) from a seeded torch
generator and quantized with the same MLX-style affine quantizer as `formats.quantize_affine`
(or OCP MXFP4 as `formats.quantize_mxfp4`), then packed in blob layout. Generating and
quantizing 16 GB of experts with numpy would take far longer than the benchmark itself.
"""
from __future__ import annotations


from . import formats as F
from .spec import LayerSpec


def quantize_affine_torch(w, group_size: int = 64, bits: int = 4):
    """(packed int32 [..., N, K*bits/32], scales bf16, biases bf16): formats.quantize_affine
    on torch tensors. Code k of a row lands at bits [bits k, bits k + bits) of the row's
    words, least significant first (a 3-bit code may straddle two words)."""
    import torch
    *lead, N, K = w.shape
    n_bins = float((1 << bits) - 1)
    g = w.float().reshape(*lead, N, K // group_size, group_size)
    w_max = g.amax(-1)
    w_min = g.amin(-1)
    mask = w_min.abs() > w_max.abs()
    scales = ((w_max - w_min) / n_bins).clamp_min(1e-7)
    scales = torch.where(mask, scales, -scales)
    edge = torch.where(mask, w_min, w_max)
    q0 = torch.round(edge / scales)
    nz = q0 != 0
    scales = torch.where(nz, edge / torch.where(nz, q0, torch.ones_like(q0)), scales)
    biases = torch.where(nz, edge, torch.zeros_like(edge))
    q = torch.clamp(torch.round((g - biases[..., None]) / scales[..., None]), 0, n_bins)
    q = q.to(torch.int64).reshape(*lead, N, K)
    if 32 % bits == 0:
        q = q.reshape(*lead, N, K * bits // 32, 32 // bits)
        shifts = torch.arange(32 // bits, device=w.device, dtype=torch.int64) * bits
        word = (q << shifts).sum(-1)
    else:
        pos = torch.arange(K, device=w.device, dtype=torch.int64) * bits
        wi, sh = pos // 32, pos % 32
        n_words = K * bits // 32
        word = torch.zeros(*lead, N, n_words, device=w.device, dtype=torch.int64)
        word.index_add_(-1, wi, (q << sh) & 0xFFFFFFFF)
        spill = torch.where(sh + bits > 32, q >> (32 - sh).clamp_max(31), torch.zeros_like(q))
        word.index_add_(-1, (wi + 1).clamp_max(n_words - 1), spill)
    word = torch.where(word >= 2 ** 31, word - 2 ** 32, word).to(torch.int32)
    return word, scales.to(torch.bfloat16), biases.to(torch.bfloat16)


def quantize_mxfp4_torch(w):
    """(packed int32 [..., N, K/8], e8m0 uint8 [..., N, K/32]): formats.quantize_mxfp4."""
    import torch
    *lead, N, K = w.shape
    g = w.float().reshape(*lead, N, K // 32, 32)
    amax = g.abs().amax(-1)
    e = torch.where(amax > 0, torch.floor(torch.log2(amax.clamp_min(1e-38))) - 2,
                    torch.full_like(amax, -127)).clamp(-127, 127)
    scaled = g / torch.exp2(e)[..., None]
    mags = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], device=w.device)
    a = scaled.abs().clamp_max(6.0)
    d = (a[..., None] - mags).abs()
    best = d.amin(-1, keepdim=True)
    cand = d == best
    idx8 = torch.arange(8, device=w.device)
    even = (idx8 % 2 == 0)
    code_even = torch.where(cand & even, idx8, torch.full_like(idx8, 99)).amin(-1)
    code_any = cand.to(torch.int64).argmax(-1)
    code = torch.where(code_even == 99, code_any, code_even)
    sign = (torch.signbit(scaled) & (code > 0)).to(torch.int64) << 3
    code = (code | sign).reshape(*lead, N, K // 8, 8)
    shifts = torch.arange(8, device=w.device, dtype=torch.int64) * 4
    word = (code << shifts).sum(-1)
    word = torch.where(word >= 2 ** 31, word - 2 ** 32, word).to(torch.int32)
    return word, (e + 127).to(torch.uint8)


def _bytes(t, E):
    import torch
    t = t.contiguous()
    if t.dtype != torch.uint8:
        t = t.view(torch.uint8)
    return t.reshape(E, -1)


def make_layer_experts(spec: LayerSpec, seed: int, std: float = 0.02, device="cuda",
                       n_experts: int | None = None, shared: bool = False):
    """uint8 [E, bytes_per_expert] on `device`: E experts of one layer in blob layout."""
    import torch
    E = n_experts or (1 if shared else spec.n_experts)
    inter = spec.shared_inter if shared else spec.inter
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    parts = []
    for proj in spec.expert_spec(shared):
        n_out, n_in = (inter, spec.hidden) if proj in ("gate_proj", "up_proj", "fc1") else (spec.hidden, inter)
        w = torch.randn((E, n_out, n_in), generator=gen, device=device, dtype=torch.float32) * std
        if spec.quant.mode == "none":
            parts.append(_bytes(w.to(torch.bfloat16), E))
        elif spec.quant.mode == "affine":
            wq, s, b = quantize_affine_torch(w, spec.quant.group_size, spec.quant.bits)
            if spec.quant.scale_dtype == "float16":
                s, b = s.float().half(), b.float().half()
            parts += [_bytes(wq, E), _bytes(s, E), _bytes(b, E)]
        else:
            wq, s = quantize_mxfp4_torch(w)
            parts += [_bytes(wq, E), _bytes(s, E)]
        del w
        if spec.has_bias:
            bias = (torch.randn((E, n_out), generator=gen, device=device) * std).to(torch.bfloat16)
            parts.append(_bytes(bias, E))
    out = torch.cat(parts, dim=1)
    want = F.spec_bytes(spec.expert_spec(shared))
    assert out.shape[1] == want, (out.shape, want)
    return out


def zipf_bias_torch(E: int, s: float, seed: int, device="cuda"):
    """-s * ln(rank + 1) over a seeded permutation of the experts (fp32 [E])."""
    import torch
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    perm = torch.randperm(E, generator=gen).to(torch.float64)
    return (-s * torch.log(perm + 1.0)).to(torch.float32).to(device)


def router_weights(spec: LayerSpec, seed: int, std: float = 0.02, device="cuda"):
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    w = torch.randn((spec.n_experts, spec.hidden), generator=gen, device=device) * std
    return w if spec.router_dtype == "float32" else w.to(torch.bfloat16)


def activations(T: int, H: int, seed: int, device="cuda"):
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return torch.randn((T, H), generator=gen, device=device).to(torch.bfloat16)


def flops_per_pair(spec: LayerSpec) -> int:
    return 2 * 3 * spec.hidden * spec.inter


