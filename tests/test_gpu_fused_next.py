"""GPU parity of the next-layer fusion (config 2's fc1 -> GELU -> fc2 and a
layer whose input concatenates two producers): the GEMM epilogue that writes
the next layer's fp6 records and fp32 low-rank partial slots, kernel 1 into
larger record / slot buffers, the fixed-order la reduction, and the module
helpers built on them.

Records must equal the act-quant kernel's on the unfused bf16 output byte
for byte (codes and scales also against the oracle's quantizer); the fp32
low-rank sums against the float64 oracle product within fp32 summation
error; final outputs within the tolerance of tests/helpers.py against the
dequantize-then-matmul oracle fed the GPU's own intermediate.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits16, check_output, decode_fp6_records
from oracle import svdq_oracle as O

from gen_worker_amd.ops import la_partials_next, la_partials_quant, records_empty

pytestmark = pytest.mark.gpu
DEV = "cuda"
REC_BYTES = 100   # codes + the two scales; bytes 100..103 of a record are unused


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import gen_worker_amd  # noqa: F401
    from gen_worker_amd import _native

    _native.load()
    assert torch.cuda.is_available()
    yield


def _layer(n, k, rank, *, smooth=True, so=0):
    from gen_worker_amd import synthetic

    return synthetic.w4a4_layer(n, k, rank, smooth=smooth, seed_offset=so)


def _act(m, k, seed):
    from gen_worker_amd import synthetic

    return synthetic.activation(m, k, outlier_frac=0.01, outlier_scale=20.0, seed=seed).to(DEV)


def _ops():
    return torch.ops.cozy_gen_worker


def _prep(down):
    return _ops().svdq_prep_proj_down_fp6(down.to(DEV)) if down is not None else None


def _dev(t):
    return t.to(DEV) if t is not None else None


def _lowrank_tol(y_bits, down_bits):
    """|fp32 sum - exact| bound: 2^-14 of the sum of |terms| (fp32 accumulation over <= 2^14 terms)."""
    ay = np.abs(O.bf16_bits_to_f32(y_bits).astype(np.float64))
    ad = np.abs(O.bf16_bits_to_f32(down_bits).astype(np.float64))
    return 2.0 ** -14 * (ay @ ad) + 1e-30


def _check_records(rec, y_bits, smooth_bits):
    """fp6 records of y against the oracle's group-64 quantizer (codes and fp16 scale bits)."""
    codes, sbits = decode_fp6_records(rec)
    qa, sa = O.quantize_act_int4(y_bits, smooth_bits)
    assert np.array_equal(O.pack_int4(codes), qa)
    assert np.array_equal(sbits, sa.view(np.uint16))


# (m, k, n, rank of this layer, rank of the next, next smooth, gelu); tile widths: 128 for the small
# grids, 256 for (1024, 512, 12288) and (2048, 256, 6272) (N % 256 == 128: a half-width last column tile)
_NEXT_CASES = [
    (77, 384, 256, 32, 32, True, True),
    (600, 256, 640, 16, 64, True, False),
    (333, 128, 3072, 0, 0, False, False),
    (1024, 512, 12288, 32, 32, True, True),
    (2048, 256, 6272, 32, 128, True, True),
    (1, 128, 384, 16, 16, True, True),
]


@pytest.mark.parametrize("m,k,n,r1,r2,sm2,gelu", _NEXT_CASES)
def test_next_epilogue_matches_unfused(m, k, n, r1, r2, sm2, gelu):
    ops = _ops()
    L1 = _layer(n, k, r1, so=m)
    L2 = _layer(128, n, r2, smooth=sm2, so=m + 1)
    x = _act(m, k, seed=m + k)
    w6 = ops.svdq_pack_weight_fp6(L1.qweight.to(DEV), L1.wscales.to(DEV))
    q6, la = ops.svdq_quant_fp6(x, _dev(L1.smooth), None, _prep(L1.proj_down))
    la = la if r1 else None
    # unfused: the bf16 output, then kernel 1 on it
    y = ops.svdq_w4a4_linear_fp6(q6, w6, None, None, la, _dev(L1.proj_up), _dev(L1.bias), torch.bfloat16, gelu)
    pdo2 = _prep(L2.proj_down)
    qn_ref, _ = ops.svdq_quant_fp6(y, _dev(L2.smooth), None, pdo2)
    # fused, into stages 2 .. 2 + n/128 of a larger buffer and the first slots of a larger partial buffer
    s = n // 128
    qn = records_empty(s + 3, m, DEV).fill_(0xAB)
    npart = la_partials_next(m, n)
    part = torch.full((npart + 1, m, r2), 7.0, device=DEV) if r2 else None
    out = ops.svdq_w4a4_linear_fp6_next(q6, w6, None, None, la, _dev(L1.proj_up), _dev(L1.bias), gelu,
                                        _dev(L2.smooth), pdo2, qn, part, 2, True)
    torch.cuda.synchronize()
    assert torch.equal(out, y)
    assert torch.equal(qn[2:2 + s, :, :REC_BYTES], qn_ref[:, :, :REC_BYTES])
    assert bool((qn[:2] == 0xAB).all()) and bool((qn[2 + s:] == 0xAB).all())
    y_bits = bits16(y.cpu())
    _check_records(qn[2:2 + s].cpu().numpy(), y_bits, bits16(L2.smooth) if sm2 else None)
    if r2:
        assert bool((part[npart] == 7.0).all())  # slots past this producer's are untouched
        d_bits = bits16(L2.proj_down)
        ref = O.lowrank_down(y_bits, d_bits)
        got = part[:npart].double().sum(0).cpu().numpy()
        assert np.all(np.abs(got - ref) <= _lowrank_tol(y_bits, d_bits)), float(np.max(np.abs(got - ref)))
        la_n = ops.svdq_la_reduce(part[:npart])
        assert la_n.dtype == torch.bfloat16 and la_n.shape == (m, r2)
        assert torch.equal(la_n, part[:npart].sum(0).to(torch.bfloat16)) or \
            float((la_n.float() - torch.from_numpy(ref).float().to(DEV)).abs().max()) <= \
            float(2.0 ** -7 * np.abs(ref).max() + 1e-6)
        # deterministic: a second run gives the same partials bit for bit
        part2 = torch.empty_like(part[:npart])
        ops.svdq_w4a4_linear_fp6_next(q6, w6, None, None, la, _dev(L1.proj_up), _dev(L1.bias), gelu,
                                      _dev(L2.smooth), pdo2, records_empty(s, m, DEV), part2, 0, False)
        assert torch.equal(part2, part[:npart])
    # without the bf16 output: the same records
    qn2 = records_empty(s, m, DEV)
    part3 = torch.empty(npart, m, r2, device=DEV) if r2 else None
    none = ops.svdq_w4a4_linear_fp6_next(q6, w6, None, None, la, _dev(L1.proj_up), _dev(L1.bias), gelu,
                                         _dev(L2.smooth), pdo2, qn2, part3, 0, False)
    torch.cuda.synchronize()
    assert none.shape == (m, 0)
    assert torch.equal(qn2[:, :, :REC_BYTES], qn_ref[:, :, :REC_BYTES])


@pytest.mark.parametrize("m,k,rank", [(77, 384, 32), (256, 3072, 32), (5, 128, 128), (300, 1024, 0),
                                      (4608, 15360, 32), (64, 12288, 64)])
def test_quant_fp6_into(m, k, rank):
    """Kernel 1 into the head of larger record / partial buffers: the same records as svdq_quant_fp6, partial
    slots that sum to x @ proj_down, the same bf16 la through svdq_la_reduce, bit for bit on a second run."""
    ops = _ops()
    L = _layer(64, k, rank, so=k)
    x = _act(m, k, seed=k)
    pdo = _prep(L.proj_down)
    q_ref, la_ref = ops.svdq_quant_fp6(x, _dev(L.smooth), None, pdo)
    s = k // 128
    q6 = records_empty(s + 2, m, DEV).fill_(0x5A)
    npart = la_partials_quant(m, k, rank) if rank else 0
    part = torch.full((npart + 1, m, rank), 3.0, device=DEV) if rank else None
    ops.svdq_quant_fp6_into(x, _dev(L.smooth), pdo, q6, part)
    torch.cuda.synchronize()
    assert torch.equal(q6[:s, :, :REC_BYTES], q_ref[:, :, :REC_BYTES])
    assert bool((q6[s:] == 0x5A).all())
    if rank:
        assert bool((part[npart] == 3.0).all())
        x_bits, d_bits = bits16(x.cpu()), bits16(L.proj_down)
        ref = O.lowrank_down(x_bits, d_bits)
        got = part[:npart].double().sum(0).cpu().numpy()
        assert np.all(np.abs(got - ref) <= _lowrank_tol(x_bits, d_bits))
        assert torch.equal(ops.svdq_la_reduce(part[:npart]), la_ref)
        q2, la2 = ops.svdq_quant_fp6(x, _dev(L.smooth), None, pdo)
        assert torch.equal(la2, la_ref) and torch.equal(q2[:, :, :REC_BYTES], q_ref[:, :, :REC_BYTES])


def _module(L, activation=None):
    from gen_worker_amd.svdq import build_svdq_w4a4_linear

    return build_svdq_w4a4_linear(qweight=L.qweight, wscales=L.wscales, smooth=L.smooth, proj_down=L.proj_down,
                                  proj_up=L.proj_up, bias=L.bias, activation=activation, device=DEV)


def _oracle(x_bits, L, gelu=False):
    return O.w4a4_linear(x_bits, bits16(L.smooth) if L.smooth is not None else None, L.qweight.numpy(),
                         L.wscales.numpy(), bits16(L.proj_down) if L.proj_down is not None else None,
                         bits16(L.proj_up) if L.proj_up is not None else None,
                         bits16(L.bias) if L.bias is not None else None, gelu=gelu)


@pytest.mark.parametrize("m,d,h,rank", [(300, 512, 1024, 32), (77, 384, 768, 16), (4608, 3072, 12288, 32)])
def test_pair_forward(m, d, h, rank):
    """svdq_pair_forward(fc1 with GELU, fc2): the fused path against fc2's oracle on the GPU's own fc1 output,
    and against the unfused module composition (which differs only by the fp32 order of la's sums)."""
    from gen_worker_amd.svdq import svdq_pair_forward

    L1, L2 = _layer(h, d, rank, so=1), _layer(d, h, rank, so=2)
    fc1, fc2 = _module(L1, "gelu_tanh"), _module(L2)
    x = _act(m, d, seed=3)
    y = svdq_pair_forward(x, fc1, fc2)
    y1 = fc1(x)
    y_unfused = fc2(y1)
    torch.cuda.synchronize()
    assert y.shape == (m, d)
    # the same records; fc2's la sums the same products grouped by fc1's column tiles instead of kernel 1's
    # K ranges, so its bf16 value may differ in the last bit
    diff = (y.float() - y_unfused.float()).abs()
    assert float(diff.max()) <= 2.0 ** -6 * float(y_unfused.float().abs().max())
    assert torch.equal(svdq_pair_forward(x, fc1, fc2), y)   # deterministic
    ref = _oracle(bits16(y1.cpu()), L2)
    check_output(y, ref, what=f"pair {m}x{d}x{h}")


@pytest.mark.parametrize("m,ka,d,h,n,rank", [(300, 384, 512, 1024, 256, 32), (4608, 3072, 3072, 12288, 3072, 32)])
def test_concat_forward(m, ka, d, h, n, rank):
    """svdq_concat_forward(consumer, a, producer, b) == consumer(cat([a, producer(b)])) against the oracle on
    the concatenation of a and the GPU's own producer output."""
    from gen_worker_amd.svdq import svdq_concat_forward

    Lp, Lc = _layer(h, d, rank, so=5), _layer(n, ka + h, rank, so=6)
    prod, cons = _module(Lp, "gelu_tanh"), _module(Lc)
    a, b = _act(m, ka, seed=7), _act(m, d, seed=8)
    y = svdq_concat_forward(cons, a, prod, b)
    yb = prod(b)
    y_unfused = cons(torch.cat((a, yb), dim=-1))
    torch.cuda.synchronize()
    assert y.shape == (m, n)
    # the same records; la's fp32 partials are grouped differently (K split at the concatenation), so the
    # bf16 la may differ in its last bit
    diff = (y.float() - y_unfused.float()).abs()
    assert float(diff.max()) <= 2.0 ** -6 * float(y_unfused.float().abs().max())
    ref = _oracle(np.concatenate((bits16(a.cpu()), bits16(yb.cpu())), axis=1), Lc)
    check_output(y, ref, what=f"concat {m} [{ka}+{h}] -> {n}")
