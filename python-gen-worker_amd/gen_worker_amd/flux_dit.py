"""Synthetic Flux-dev-shaped DiT denoiser: the config-4 workload of the benchmark.

One denoising forward at batch 1, 1024 x 1024 (4096 image tokens of 64 latent
channels + 512 text tokens of 4096 T5 features), 19 dual-stream and 38
single-stream blocks, hidden 3072, 24 heads of 128, MLP ratio 4: the block
structure of diffusers' ``FluxTransformer2DModel`` (AdaLayerNormZero
modulation, joint attention over [text; image] with RMSNorm on q/k and rotary
embeddings, GELU-tanh MLPs; single blocks run attention and the MLP side by
side and project their concatenation). The timestep / guidance / pooled-text
conditioning enters as a seeded random embedding ``temb`` [1, 3072].

Every linear is built by a factory, so the same model runs as:
  * ``"w4a4"``: every linear an SVDQuant W4A4 layer (``SvdqW4A4Linear``,
    rank 32, group 64; int4 codes, fp16 scales, low-rank factors and bias
    random), GELU fused into the fc1 epilogues, and each MLP's second linear
    quantized in the first one's epilogue (``svdq_pair_forward``; in the
    single blocks ``svdq_concat_forward`` builds proj_out's input [attention,
    MLP] without the concatenation). The blocks' adaLN modulation linears
    (one token) are W4A4 too, or with ``modulation="awq"`` AWQ W4A16
    (``AwqPackedLinear``), the format an svdq checkpoint keeps them in. The
    int4 layers follow the process's qualified lane (``qualify.resolve_lane``,
    or ``lane=`` to pin it): in the dense lane each is served as its folded
    bf16 Linear, as the reference's swap does;
  * ``"bf16"``: every linear a bf16 ``nn.Linear`` (the bf16 GEMM path).
Both models share the rest of the block: the fused glue kernels below (q/k
RMSNorm + rotary, adaLN modulation, gated residual) and the attention, chosen
per model: ``attention="sdpa"`` (the default) is diffusers' call, torch's bf16
scaled_dot_product_attention restricted to its flash / memory-efficient
kernels; ``attention="flash"`` is this package's bf16 flash-attention kernel
(``gwa_dit_attention``). Weights are random-init on the device from seeded
generators; values are chosen only to keep activations finite and O(1)
through the 57 blocks.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .graphs import capture_graph


@dataclass(frozen=True)
class FluxDiTConfig:
    hidden: int = 3072
    heads: int = 24
    head_dim: int = 128
    mlp: int = 12288
    n_dual: int = 19
    n_single: int = 38
    img_tokens: int = 4096
    txt_tokens: int = 512
    in_channels: int = 64
    txt_dim: int = 4096
    rank: int = 32


def _w4a4_linear(in_f: int, out_f: int, seed: int, device, rank: int, gelu: bool = False) -> nn.Module:
    """A random-init SvdqW4A4Linear: uniform int4 codes, fp16 group scales with effective weight std ~0.02,
    smoothing factors log-uniform in [0.5, 2], L1 / L2 / bias ~ N(0, 0.02)."""
    from .svdq import SvdqW4A4Linear

    g = torch.Generator(device=device).manual_seed(seed)
    mod = SvdqW4A4Linear(in_f, out_f, rank=rank, bias=True, activation="gelu_tanh" if gelu else None,
                         device=device)
    with torch.no_grad():
        mod.weight.copy_(torch.randint(0, 256, mod.weight.shape, generator=g, device=device, dtype=torch.int32)
                         .to(torch.uint8))
        # uniform codes in [-8, 7] have std ~4.6: scale for an effective weight std of ~0.02
        sc = 0.02 / 4.61 * (0.75 + 0.5 * torch.rand(mod.weight_scale.shape, generator=g, device=device))
        mod.weight_scale.copy_(sc.to(torch.float16))
        u = torch.rand(in_f, generator=g, device=device)
        mod.smooth_factor.copy_(torch.exp(math.log(0.5) + u * math.log(4.0)).to(torch.bfloat16))
        if rank:
            mod.proj_down.copy_(torch.randn(in_f, rank, generator=g, device=device).mul_(0.02).to(torch.bfloat16))
            mod.proj_up.copy_(torch.randn(out_f, rank, generator=g, device=device).mul_(0.02).to(torch.bfloat16))
        mod.bias.copy_(torch.randn(out_f, generator=g, device=device).mul_(0.02).to(torch.bfloat16))
    mod.refresh_derived()
    return mod


def _awq_linear(in_f: int, out_f: int, seed: int, device) -> nn.Module:
    """A random-init AWQ W4A16 modulation linear: uniform uint4 codes, bf16 group scales for an effective
    weight std of ~0.02 and zeros centring the codes (w = code * s + z ~ 0 on average), bias ~ N(0, 0.02)."""
    from .awq import AwqPackedLinear

    g = torch.Generator(device=device).manual_seed(seed)
    mod = AwqPackedLinear(in_f, out_f, bias=True, device=device)
    with torch.no_grad():
        mod.weight.copy_(torch.randint(0, 256, mod.weight.shape, generator=g, device=device, dtype=torch.int32)
                         .to(torch.uint8))
        sc = 0.02 / 4.61 * (0.75 + 0.5 * torch.rand(mod.wscales.shape, generator=g, device=device))
        mod.wscales.copy_(sc.to(torch.bfloat16))
        mod.wzeros.copy_((-7.5 * sc).to(torch.bfloat16))
        mod.bias.copy_(torch.randn(out_f, generator=g, device=device).mul_(0.02).to(torch.bfloat16))
    return mod


class _Bf16Linear(nn.Module):
    """bf16 nn.Linear (weights ~ N(0, 0.02)) with the same optional GELU-tanh as the fused lane."""

    def __init__(self, in_f: int, out_f: int, seed: int, device, gelu: bool = False) -> None:
        super().__init__()
        g = torch.Generator(device=device).manual_seed(seed)
        self.lin = nn.Linear(in_f, out_f, bias=True, device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            self.lin.weight.copy_(torch.randn(out_f, in_f, generator=g, device=device).mul_(0.02))
            self.lin.bias.copy_(torch.randn(out_f, generator=g, device=device).mul_(0.02))
        self.gelu = gelu

    def forward(self, x: Tensor) -> Tensor:
        y = self.lin(x)
        return F.gelu(y, approximate="tanh") if self.gelu else y


def linear_factory(kind: str, device, rank: int, lane: str = "int4") -> Callable[..., nn.Module]:
    """``make(in_f, out_f, seed, gelu=False)`` for ``kind`` in ("w4a4", "bf16"); a "w4a4" layer in the dense
    lane is served as its fold."""
    if kind == "w4a4":
        from .qualify import serving_linear

        return lambda i, o, s, gelu=False: serving_linear(_w4a4_linear(i, o, s, device, rank, gelu), lane)
    if kind == "bf16":
        return lambda i, o, s, gelu=False: _Bf16Linear(i, o, s, device, gelu)
    raise ValueError(f"linear kind {kind!r} not in ('w4a4', 'bf16')")


MODULATIONS = ("w4a4", "awq")


def modulation_factory(kind: str, device, rank: int = 32, lane: str = "int4",
                       modulation: str = "w4a4") -> Callable[..., nn.Module]:
    """``make(in_f, out_f, seed)`` for the adaLN modulation linears (one token): in the "w4a4" model W4A4
    layers like every other linear, or with ``modulation="awq"`` AWQ W4A16 through the AWQ GEMV (an svdq
    checkpoint keeps them in that format, ``models/svdq_awq.py:1``); "bf16" keeps bf16 linears."""
    if modulation not in MODULATIONS:
        raise ValueError(f"modulation {modulation!r} not in {MODULATIONS}")
    if kind == "w4a4" and modulation == "w4a4":
        make = linear_factory(kind, device, rank, lane)
        return lambda i, o, s: make(i, o, s)
    if kind == "w4a4":
        return lambda i, o, s: _awq_linear(i, o, s, device)
    if kind == "bf16":
        return lambda i, o, s: _Bf16Linear(i, o, s, device)
    raise ValueError(f"linear kind {kind!r} not in ('w4a4', 'bf16')")


# torch statements of the block glue; the blocks run the fused kernels below (csrc/dit_block.hip), which
# round every step as these expressions do
def _rms(x: Tensor, w: Tensor, eps: float = 1e-6) -> Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w


def _ln(x: Tensor) -> Tensor:
    return F.layer_norm(x, (x.shape[-1],), eps=1e-6)


def _rope(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Rotary embedding on interleaved (even, odd) pairs: x [S, H, D], cos / sin [S, 1, D/2]."""
    xe, xo = x[..., 0::2], x[..., 1::2]
    return torch.stack((xe * cos - xo * sin, xe * sin + xo * cos), dim=-1).flatten(-2)


def _check_rows(name: str, t: Tensor, cols: int) -> None:
    if t.dtype != torch.bfloat16 or not t.is_cuda:
        raise ValueError(f"{name}: bf16 CUDA tensor expected, got {t.dtype} on {t.device}")
    if t.dim() != 2 or t.shape[1] != cols or t.stride(1) != 1:
        raise ValueError(f"{name}: [rows, {cols}] with unit column stride expected, got {tuple(t.shape)} "
                         f"strides {t.stride()}")


def _vector(name: str, t: Tensor, cols: int) -> Tensor:
    v = t.reshape(-1)
    if v.numel() != cols or v.dtype != torch.bfloat16 or (cols > 1 and v.stride(0) != 1):
        raise ValueError(f"{name}: {cols} contiguous bf16 values expected, got {tuple(t.shape)} {t.dtype}")
    return v


def adaln_modulate(x: Tensor, scale: Tensor, shift: Tensor, eps: float = 1e-6) -> Tensor:
    """``_ln(x) * (1 + scale) + shift`` in one pass (``gwa_dit_adaln_modulate``): x bf16 [rows, C] (row
    stride allowed), scale / shift C bf16 values (e.g. chunks of a modulation output)."""
    from . import _native

    c = x.shape[-1]
    _check_rows("adaln_modulate x", x, c)
    sc, sh = _vector("adaln_modulate scale", scale, c), _vector("adaln_modulate shift", shift, c)
    out = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    _native.call("gwa_dit_adaln_modulate", _native.ptr(x), x.stride(0), _native.ptr(sc), _native.ptr(sh),
                 _native.ptr(out), c, x.shape[0], c, eps, _native.stream_of(x))
    return out


def gate_residual(x: Tensor, y: Tensor, gate: Tensor) -> Tensor:
    """``x + gate * y`` in one pass (``gwa_dit_gate_residual``): x, y bf16 [rows, C], gate C bf16 values
    broadcast over rows."""
    from . import _native

    c = x.shape[-1]
    _check_rows("gate_residual x", x, c)
    _check_rows("gate_residual y", y, c)
    if y.shape[0] != x.shape[0]:
        raise ValueError(f"gate_residual: x has {x.shape[0]} rows, y {y.shape[0]}")
    g = _vector("gate_residual gate", gate, c)
    out = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    _native.call("gwa_dit_gate_residual", _native.ptr(x), x.stride(0), _native.ptr(y), y.stride(0), _native.ptr(g),
                 _native.ptr(out), c, x.shape[0], c, _native.stream_of(x))
    return out


def qk_norm_rope(q: Tensor, k: Tensor, wq: Tensor, wk: Tensor, cos: Tensor, sin: Tensor, pos0: int,
                 out_q: Tensor, out_k: Tensor, v: Optional[Tensor] = None, out_v: Optional[Tensor] = None,
                 eps: float = 1e-6) -> None:
    """``_rope(_rms(q, wq), cos, sin)`` and the same for k, in one pass (``gwa_dit_qk_norm_rope``), written
    into out_q / out_k [rows, heads, 128] (row slices of a joint sequence's buffers); v, if given, is copied to
    out_v. q, k (, v): [rows, heads * 128] views sharing one row stride (column slices of a fused qkv output);
    the rotary tables cos / sin [positions, 1, 64] are read at positions pos0 + row."""
    from . import _native

    rows, heads, d = out_q.shape
    hd = heads * d
    for name, t in (("q", q), ("k", k)) + ((("v", v),) if v is not None else ()):
        _check_rows(f"qk_norm_rope {name}", t, hd)
        if t.shape[0] != rows or t.stride(0) != q.stride(0):
            raise ValueError(f"qk_norm_rope {name}: {rows} rows at q's row stride expected")
    outs = (out_q, out_k) + ((out_v,) if out_v is not None else ())
    for o in outs:
        if o.shape != out_q.shape or o.stride() != out_q.stride() or o.stride(1) != d or o.stride(2) != 1:
            raise ValueError("qk_norm_rope: outputs must be [rows, heads, head_dim] with rows at one stride")
    if (v is None) != (out_v is None):
        raise ValueError("qk_norm_rope: v and out_v go together")
    if cos.shape != sin.shape or not cos.is_contiguous() or not sin.is_contiguous() or cos.shape[-1] * 2 != d:
        raise ValueError("qk_norm_rope: cos / sin must be contiguous [positions, 1, head_dim / 2] tables")
    wq, wk = _vector("qk_norm_rope wq", wq, d), _vector("qk_norm_rope wk", wk, d)
    _native.call("gwa_dit_qk_norm_rope", _native.ptr(q), _native.ptr(k), _native.ptr(v), q.stride(0),
                 _native.ptr(wq), _native.ptr(wk), _native.ptr(cos), _native.ptr(sin), pos0, cos.shape[0],
                 _native.ptr(out_q), _native.ptr(out_k), _native.ptr(out_v), out_q.stride(0), rows, heads, d, eps,
                 _native.stream_of(out_q))


def _sdpa(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """torch's statement of the block attention: [S, H, D] bf16 -> [S, H*D] via SDPA on [1, H, S, D] (any
    backend torch picks)."""
    s, h, d = q.shape
    o = F.scaled_dot_product_attention(q.transpose(0, 1).unsqueeze(0), k.transpose(0, 1).unsqueeze(0),
                                       v.transpose(0, 1).unsqueeze(0))
    return o.squeeze(0).transpose(0, 1).reshape(s, h * d)


def sdpa_attention(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """The block attention as diffusers calls it (``F.scaled_dot_product_attention`` on [1, H, S, D] bf16),
    restricted to torch's flash and memory-efficient kernels: the math fallback (batched bf16 products on
    transposed views) is never taken; a shape those kernels refuse raises instead."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return _sdpa(q, k, v)


def attention(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """Joint self-attention of a block (``gwa_dit_attention``): q, k, v bf16 [S, H, 128] with unit head and
    element strides (token strides free: v may be a column slice of a fused qkv output) -> [S, H * 128]."""
    from . import _native

    s, h, d = q.shape
    for name, t in (("q", q), ("k", k), ("v", v)):
        if (t.dtype != torch.bfloat16 or not t.is_cuda or t.dim() != 3 or tuple(t.shape[1:]) != (h, d)
                or t.stride(2) != 1 or t.stride(1) != d):
            raise ValueError(f"attention {name}: bf16 CUDA [tokens, {h}, {d}] with unit head / element strides "
                             f"expected, got {tuple(t.shape)} strides {t.stride()} {t.dtype}")
    if k.shape[0] != v.shape[0]:
        raise ValueError(f"attention: {k.shape[0]} keys, {v.shape[0]} values")
    out = torch.empty(s, h * d, device=q.device, dtype=torch.bfloat16)
    _native.call("gwa_dit_attention", _native.ptr(q), q.stride(0), _native.ptr(k), k.stride(0), _native.ptr(v),
                 v.stride(0), _native.ptr(out), h * d, s, k.shape[0], h, d, 1.0 / math.sqrt(d),
                 _native.stream_of(q))
    return out


ATTENTION = {"sdpa": sdpa_attention, "flash": attention}


def _mlp(fc1: nn.Module, fc2: nn.Module, x: Tensor, fused: bool) -> Tensor:
    if fused:
        from .svdq import svdq_pair_forward

        return svdq_pair_forward(x, fc1, fc2)
    return fc2(fc1(x))


def _take_modulation(blk: nn.Module, compute: Callable[[], tuple]) -> tuple:
    """The block's modulation outputs: precomputed on another stream (``pre_mod`` = (outputs, event): this stream
    waits for the event), or computed here."""
    pre = blk.pre_mod
    if pre is None:
        return compute()
    outs, ev = pre
    blk.pre_mod = None
    torch.cuda.current_stream(outs[0].device).wait_event(ev)
    return outs


class DualBlock(nn.Module):
    def __init__(self, cfg: FluxDiTConfig, make, seed: int, device, fused: bool = False, make_mod=None) -> None:
        super().__init__()
        c = cfg.hidden
        self.cfg, self.fused = cfg, fused
        make_mod = make_mod or (lambda i, o, s: make(i, o, s))
        self.mod_img, self.mod_txt = make_mod(c, 6 * c, seed), make_mod(c, 6 * c, seed + 1)
        self.qkv_img, self.qkv_txt = make(c, 3 * c, seed + 2), make(c, 3 * c, seed + 3)
        self.o_img, self.o_txt = make(c, c, seed + 4), make(c, c, seed + 5)
        self.fc1_img, self.fc1_txt = make(c, cfg.mlp, seed + 6, gelu=True), make(c, cfg.mlp, seed + 7, gelu=True)
        self.fc2_img, self.fc2_txt = make(cfg.mlp, c, seed + 8), make(cfg.mlp, c, seed + 9)
        self.side: Optional[torch.cuda.Stream] = None  # set by FluxDiT(..., streams=2)
        self.attn: Callable[[Tensor, Tensor, Tensor], Tensor] = sdpa_attention  # set by FluxDiT(..., attention=)
        self.pre_mod = None  # modulation outputs computed ahead on another stream, and their event
        ones = torch.ones(cfg.head_dim, device=device, dtype=torch.bfloat16)
        self.register_buffer("qn_img", ones.clone())
        self.register_buffer("kn_img", ones.clone())
        self.register_buffer("qn_txt", ones.clone())
        self.register_buffer("kn_txt", ones.clone())

    def forward(self, img: Tensor, txt: Tensor, temb: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
        if self.side is not None:
            return self._forward_two_streams(img, txt, temb, cos, sin)
        cfg = self.cfg
        mi, mt = _take_modulation(self, lambda: (self.mod_img(temb), self.mod_txt(temb)))
        sh1, sc1, g1, sh2, sc2, g2 = mi.chunk(6, dim=-1)
        tsh1, tsc1, tg1, tsh2, tsc2, tg2 = mt.chunk(6, dim=-1)
        c, st = cfg.hidden, txt.shape[0]
        qkv_i = self.qkv_img(adaln_modulate(img, sc1, sh1))
        qkv_t = self.qkv_txt(adaln_modulate(txt, tsc1, tsh1))
        # q, k, v of the joint [text; image] sequence, written in place by the norm + rotary kernel
        q, k, v = (torch.empty(st + img.shape[0], cfg.heads, cfg.head_dim, device=img.device, dtype=img.dtype)
                   for _ in range(3))
        for src, qn, kn, rows in ((qkv_t, self.qn_txt, self.kn_txt, slice(0, st)),
                                  (qkv_i, self.qn_img, self.kn_img, slice(st, None))):
            qk_norm_rope(src[:, :c], src[:, c:2 * c], qn, kn, cos, sin, rows.start, q[rows], k[rows],
                         v=src[:, 2 * c:], out_v=v[rows])
        a = self.attn(q, k, v)
        at, ai = a[:st], a[st:]
        img = gate_residual(img, self.o_img(ai.contiguous()), g1)
        txt = gate_residual(txt, self.o_txt(at.contiguous()), tg1)
        img = gate_residual(img, _mlp(self.fc1_img, self.fc2_img, adaln_modulate(img, sc2, sh2), self.fused), g2)
        txt = gate_residual(txt, _mlp(self.fc1_txt, self.fc2_txt, adaln_modulate(txt, tsc2, tsh2), self.fused),
                            tg2)
        return img, txt

    def _forward_two_streams(self, img: Tensor, txt: Tensor, temb: Tensor, cos: Tensor,
                             sin: Tensor) -> tuple[Tensor, Tensor]:
        """The same kernels on the same inputs, the text stream's (512 tokens: grids that leave CUs idle) on a
        second HIP stream, joined for the attention and at the end."""
        cfg, side = self.cfg, self.side
        main = torch.cuda.current_stream(img.device)
        c, st = cfg.hidden, txt.shape[0]
        pre = self.pre_mod is not None
        if pre:
            mi, mt = _take_modulation(self, None)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            if not pre:
                mt = self.mod_txt(temb)
            tsh1, tsc1, tg1, tsh2, tsc2, tg2 = mt.chunk(6, dim=-1)
            qkv_t = self.qkv_txt(adaln_modulate(txt, tsc1, tsh1))
        if not pre:
            mi = self.mod_img(temb)
        sh1, sc1, g1, sh2, sc2, g2 = mi.chunk(6, dim=-1)
        qkv_i = self.qkv_img(adaln_modulate(img, sc1, sh1))
        q, k, v = (torch.empty(st + img.shape[0], cfg.heads, cfg.head_dim, device=img.device, dtype=img.dtype)
                   for _ in range(3))
        side.wait_stream(main)  # q, k, v allocated before the text rows are written on the side stream
        with torch.cuda.stream(side):
            qk_norm_rope(qkv_t[:, :c], qkv_t[:, c:2 * c], self.qn_txt, self.kn_txt, cos, sin, 0, q[:st], k[:st],
                         v=qkv_t[:, 2 * c:], out_v=v[:st])
        qk_norm_rope(qkv_i[:, :c], qkv_i[:, c:2 * c], self.qn_img, self.kn_img, cos, sin, st, q[st:], k[st:],
                     v=qkv_i[:, 2 * c:], out_v=v[st:])
        # the joint attention as two launches over the same keys: the text queries' on the side stream (its
        # 96 workgroups finish in the first round, so the text stream's next kernels can take the CUs the
        # image queries' last round leaves idle), the image queries' here; each query's result is the same
        main.wait_stream(side)
        side.wait_stream(main)
        ai = self.attn(q[st:], k, v)
        with torch.cuda.stream(side):
            at = self.attn(q[:st], k, v)
            t2 = gate_residual(txt, self.o_txt(at), tg1)
            t2 = gate_residual(t2, _mlp(self.fc1_txt, self.fc2_txt, adaln_modulate(t2, tsc2, tsh2), self.fused),
                               tg2)
        img = gate_residual(img, self.o_img(ai.contiguous()), g1)
        img = gate_residual(img, _mlp(self.fc1_img, self.fc2_img, adaln_modulate(img, sc2, sh2), self.fused), g2)
        # joined before any tensor of this block is freed: the allocator's per-stream pools stay ordered (a
        # block freed here is reused only after this join, or by the stream that allocated it)
        main.wait_stream(side)
        return img, t2


class SingleBlock(nn.Module):
    def __init__(self, cfg: FluxDiTConfig, make, seed: int, device, fused: bool = False, make_mod=None) -> None:
        super().__init__()
        c = cfg.hidden
        self.cfg, self.fused = cfg, fused
        make_mod = make_mod or (lambda i, o, s: make(i, o, s))
        self.mod = make_mod(c, 3 * c, seed)
        self.qkv = make(c, 3 * c, seed + 1)
        self.mlp = make(c, cfg.mlp, seed + 2, gelu=True)
        self.proj_out = make(c + cfg.mlp, c, seed + 3)
        self.side: Optional[torch.cuda.Stream] = None  # set by FluxDiT(..., streams=2)
        self.attn: Callable[[Tensor, Tensor, Tensor], Tensor] = sdpa_attention  # set by FluxDiT(..., attention=)
        self.pre_mod = None
        ones = torch.ones(cfg.head_dim, device=device, dtype=torch.bfloat16)
        self.register_buffer("qn", ones.clone())
        self.register_buffer("kn", ones.clone())

    def forward(self, x: Tensor, temb: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
        cfg = self.cfg
        (m3,) = _take_modulation(self, lambda: (self.mod(temb),))
        sh, sc, g = m3.chunk(3, dim=-1)
        n = adaln_modulate(x, sc, sh)
        c = cfg.hidden
        side = self.side
        if side is not None:
            # the MLP branch (it needs only n) on the second stream while the attention branch runs here;
            # joined before proj_out reads both
            main = torch.cuda.current_stream(x.device)
            if self.fused:
                from .svdq import SvdqConcat

                cc = SvdqConcat(self.proj_out, self.mlp, n, c)  # buffers allocated on this stream first
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    cc.produce()
            else:
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    h = self.mlp(n)
        qkv = self.qkv(n)
        q, k = (torch.empty(x.shape[0], cfg.heads, cfg.head_dim, device=x.device, dtype=x.dtype) for _ in range(2))
        qk_norm_rope(qkv[:, :c], qkv[:, c:2 * c], self.qn, self.kn, cos, sin, 0, q, k)
        a = self.attn(q, k, qkv[:, 2 * c:].reshape(-1, cfg.heads, cfg.head_dim))
        if side is not None:
            if self.fused:
                return gate_residual(x, cc.finish(a, before_reduce=lambda: main.wait_stream(side)), g)
            main.wait_stream(side)
            return gate_residual(x, self.proj_out(torch.cat((a, h), dim=-1)), g)
        if self.fused:
            from .svdq import svdq_concat_forward

            return gate_residual(x, svdq_concat_forward(self.proj_out, a, self.mlp, n), g)
        return gate_residual(x, self.proj_out(torch.cat((a, self.mlp(n)), dim=-1)), g)


class FluxDiT(nn.Module):
    """The config-4 denoiser; ``forward(latents [4096, 64], text [512, 4096], temb [1, 3072]) -> [4096, 64]``.
    ``attention``: ``"sdpa"`` (torch's SDPA, as config 4 states) or ``"flash"`` (``gwa_dit_attention``)."""

    def __init__(self, kind: str, cfg: FluxDiTConfig = FluxDiTConfig(), device="cuda", seed: int = 1000,
                 lane: Optional[str] = None, modulation: str = "w4a4", streams: int = 1,
                 attention: str = "sdpa") -> None:
        super().__init__()
        if attention not in ATTENTION:
            raise ValueError(f"attention must be one of {sorted(ATTENTION)}, got {attention!r}")
        self.attention = attention
        if kind == "w4a4":
            from .qualify import resolve_lane

            self.lane = resolve_lane(lane)
        else:
            self.lane = "bf16"
        make = linear_factory(kind, device, cfg.rank, self.lane)
        make_mod = modulation_factory(kind, device, cfg.rank, self.lane, modulation)
        self.cfg, self.kind, self.modulation = cfg, kind, modulation
        c = cfg.hidden
        self.x_embedder = make(cfg.in_channels, c, seed)
        self.context_embedder = make(cfg.txt_dim, c, seed + 1)
        fused = self.lane == "int4"
        self.dual = nn.ModuleList(DualBlock(cfg, make, seed + 100 + 10 * i, device, fused, make_mod)
                                  for i in range(cfg.n_dual))
        self.single = nn.ModuleList(SingleBlock(cfg, make, seed + 400 + 10 * i, device, fused, make_mod)
                                    for i in range(cfg.n_single))
        for blk in list(self.dual) + list(self.single):
            blk.attn = ATTENTION[attention]
        self.mod_stream: Optional[torch.cuda.Stream] = None
        if streams == 2:  # a second HIP stream (default priority): the dual blocks' text stream, the single
            side = torch.cuda.Stream(device=device)  # blocks' MLP branch
            for blk in list(self.dual) + list(self.single):
                blk.side = side
            # and a third for the modulation linears (they read only the timestep embedding): all of them are
            # queued there at the start, each block waiting for its own
            self.mod_stream = torch.cuda.Stream(device=device)
        elif streams != 1:
            raise ValueError(f"streams must be 1 or 2, got {streams}")
        self.norm_out = make(c, 2 * c, seed + 2)
        self.proj_out = make(c, cfg.in_channels, seed + 3)
        # rotary tables for the 4608 joint positions ([text; image]), theta 10000
        s = cfg.txt_tokens + cfg.img_tokens
        half = cfg.head_dim // 2
        inv = 1.0 / (10000.0 ** (torch.arange(half, device=device, dtype=torch.float32) / half))
        ang = torch.arange(s, device=device, dtype=torch.float32)[:, None] * inv[None, :]
        self.register_buffer("cos", ang.cos().to(torch.bfloat16).unsqueeze(1))
        self.register_buffer("sin", ang.sin().to(torch.bfloat16).unsqueeze(1))

    def forward(self, latents: Tensor, text: Tensor, temb: Tensor) -> Tensor:
        t = F.silu(temb)
        ms = self.mod_stream
        if ms is not None:
            main = torch.cuda.current_stream(t.device)
            ms.wait_stream(main)
            with torch.cuda.stream(ms):
                for blk in self.dual:
                    outs = (blk.mod_img(t), blk.mod_txt(t))
                    ev = torch.cuda.Event()
                    ev.record(ms)
                    blk.pre_mod = (outs, ev)
                for blk in self.single:
                    outs = (blk.mod(t),)
                    ev = torch.cuda.Event()
                    ev.record(ms)
                    blk.pre_mod = (outs, ev)
                nmod = self.norm_out(t)
        img = self.x_embedder(latents)
        txt = self.context_embedder(text)
        for blk in self.dual:
            img, txt = blk(img, txt, t, self.cos, self.sin)
        x = torch.cat((txt, img))
        for blk in self.single:
            x = blk(x, t, self.cos, self.sin)
        img = x[self.cfg.txt_tokens:]
        if ms is not None:
            main.wait_stream(ms)  # the last modulation; every tensor the stream wrote is consumed after this
            scale, shift = nmod.chunk(2, dim=-1)
        else:
            scale, shift = self.norm_out(t).chunk(2, dim=-1)
        return self.proj_out(adaln_modulate(img, scale, shift))


def inputs(cfg: FluxDiTConfig = FluxDiTConfig(), device="cuda", seed: int = 7) -> tuple[Tensor, Tensor, Tensor]:
    """Seeded (latents [4096, 64], text features [512, 4096], temb [1, 3072]) in bf16."""
    g = torch.Generator(device=device).manual_seed(seed)
    lat = torch.randn(cfg.img_tokens, cfg.in_channels, generator=g, device=device).to(torch.bfloat16)
    txt = torch.randn(cfg.txt_tokens, cfg.txt_dim, generator=g, device=device).to(torch.bfloat16)
    temb = torch.randn(1, cfg.hidden, generator=g, device=device).to(torch.bfloat16)
    return lat, txt, temb


def block_int_ops(cfg: FluxDiTConfig = FluxDiTConfig()) -> int:
    """2 * M * N * K of every block linear (the modulation / embedding linears excluded)."""
    c, m4, s = cfg.hidden, cfg.mlp, cfg.img_tokens + cfg.txt_tokens
    per_stream = c * 3 * c + c * c + c * m4 + m4 * c
    dual = 2 * (cfg.img_tokens + cfg.txt_tokens) * per_stream
    single = 2 * s * (c * 3 * c + c * m4 + (c + m4) * c)
    return cfg.n_dual * dual + cfg.n_single * single


def time_step_ms(model: nn.Module, args: tuple[Tensor, ...], steps: int = 5, warmup: int = 2,
                 graph: bool = True) -> float:
    """Mean ms per forward, replaying ``steps`` forwards captured in one HIP graph (or eager)."""
    with torch.no_grad():
        for _ in range(warmup):
            model(*args)
        torch.cuda.synchronize()
        if graph:
            g, out = capture_graph(lambda: model(*args))
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            del out
            return e0.elapsed_time(e1) / steps
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            model(*args)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps


__all__ = ["ATTENTION", "FluxDiT", "FluxDiTConfig", "adaln_modulate", "attention", "block_int_ops", "gate_residual",
           "inputs", "linear_factory", "qk_norm_rope", "sdpa_attention", "time_step_ms"]
