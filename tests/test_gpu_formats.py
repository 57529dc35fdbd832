"""GPU parity of the other weight formats (csrc/formats.hip) against oracle/formats.py (run with -m gpu).

* the FP8 E4M3 per-row and INT4 per-group quantizers equal the oracle bit for bit
  (codes, packed nibbles and scales), on random rows and edge rows;
* the FP8 and INT4 matvecs are within 1e-5 relative L2 of the float64 product of
  the oracle's dequantized weights, at the config-2 shapes and at ragged ones;
  an FP8 matrix drawn over every finite code checks the hardware decode of each;
* their steady-state forms give every copy's product.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import formats as of

pytestmark = pytest.mark.gpu

CONFIG2 = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (151936, 1024)]


def _weights(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16)
    if M > 4:
        w[1] = 0                                    # zero row: scale floor
        w[2, 0] = -3.0                              # one large element
        w[3, ::2] = 0.5                             # many equal magnitudes
        w[4] = -w[4]
    return w


def _rel(got, ref):
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300))


@pytest.mark.parametrize("shape", [(4096, 1024), (1024, 3072), (37, 48), (5, 100), (3, 16)], ids=str)
def test_fp8_quantize_bit_exact(mq, dev, shape):
    print(f"fp8 quantize {shape}", flush=True)
    w = _weights(*shape, seed=shape[0] + 3 * shape[1])
    q, s = mq.quantize_fp8(w.to(dev))
    qr, sr = of.quantize_fp8_rows(w)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu(), qr)


@pytest.mark.parametrize("shape", [(4096, 1024), (1024, 3072), (19, 512), (1, 128), (7, 16384)], ids=str)
def test_int4_quantize_bit_exact(mq, dev, shape):
    print(f"int4 quantize {shape}", flush=True)
    w = _weights(*shape, seed=shape[0] + 5 * shape[1])
    q, s = mq.quantize_int4(w.to(dev))
    qr, sr = of.quantize_int4_groups(w)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu(), qr)


@pytest.mark.parametrize("shape", CONFIG2 + [(1, 16), (37, 48), (300, 2064), (3, 16384), (1000, 8192)], ids=str)
def test_fp8_gemv_parity(mq, dev, shape):
    M, K = shape
    print(f"fp8 gemv {M}x{K}", flush=True)
    w = _weights(M, K, seed=M + 7 * K)
    q, s = of.quantize_fp8_rows(w)
    x = torch.randn(K, generator=torch.Generator().manual_seed(K), dtype=torch.float32)
    y = mq.fp8_gemv(x.to(dev), q.to(dev), s.to(dev))
    torch.cuda.synchronize()
    ref = of.matvec_f64(of.dequant_fp8(q, s), x)
    assert _rel(y.cpu().double().numpy(), ref) <= 1e-5


def test_fp8_gemv_every_code(mq, dev):
    """Codes drawn over all 254 finite values (subnormals and +-448 included), so every code's
    hardware decode enters a product."""
    M, K = 512, 1024
    g = torch.Generator().manual_seed(8)
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=torch.uint8)
    q = codes[torch.randint(0, len(codes), (M, K), generator=g)]
    q[0, :254] = codes                                   # each code at least once
    s = torch.rand(M, generator=g) * 1e-3 + 1e-4
    x = torch.randn(K, generator=g)
    y = mq.fp8_gemv(x.to(dev), q.to(dev), s.to(dev))
    torch.cuda.synchronize()
    ref = of.matvec_f64(of.dequant_fp8(q, s), x)
    assert _rel(y.cpu().double().numpy(), ref) <= 1e-5
    # one-hot activations read single codes back: every finite code decodes exactly
    for k in (0, 100, 253):
        e = torch.zeros(K)
        e[k] = 1.0
        yk = mq.fp8_gemv(e.to(dev), q.to(dev), torch.ones(M).to(dev)).cpu().double().numpy()
        assert np.array_equal(yk, of.fp8_decode_table()[q[:, k].numpy().astype(np.int64)])


@pytest.mark.parametrize("shape", CONFIG2 + [(1, 128), (37, 128), (300, 2176), (3, 16384), (1000, 8192)], ids=str)
def test_int4_gemv_parity(mq, dev, shape):
    M, K = shape
    print(f"int4 gemv {M}x{K}", flush=True)
    w = _weights(M, K, seed=M + 11 * K)
    q, s = of.quantize_int4_groups(w)
    x = torch.randn(K, generator=torch.Generator().manual_seed(K + 1), dtype=torch.float32)
    y = mq.int4_gemv(x.to(dev), q.to(dev), s.to(dev))
    torch.cuda.synchronize()
    ref = of.matvec_f64(of.dequant_int4(q, s), x)
    assert _rel(y.cpu().double().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("shape", [(64, 1024), (40, 384)], ids=str)
def test_int4_gemv_one_hot_and_scale_layouts(mq, dev, shape):
    """One-hot activations read single dequantized weights back exactly (s * q is exact in
    fp32), at unit, tiny and negative magnitudes; and scales not 16-byte aligned (read one
    group at a time) give the same result as aligned ones (read four groups at a time)."""
    M, K = shape
    print(f"int4 gemv one-hot / scale layouts {M}x{K}", flush=True)
    q, s = of.quantize_int4_groups(_weights(M, K, seed=7 + K))
    deq = np.asarray(of.dequant_int4(q, s), dtype=np.float64)
    qd, sd = q.to(dev), s.to(dev)
    for k, v in ((0, 1.0), (K // 2 + 3, -1.0), (K - 1, 2.0 ** -100), (129 % K, -3.0 * 2.0 ** 90)):
        e = torch.zeros(K)
        e[k] = v
        yk = mq.int4_gemv(e.to(dev), qd, sd).cpu().double().numpy()
        assert np.array_equal(yk, (deq[:, k] * v).astype(np.float32).astype(np.float64)), (k, v)
    x = torch.randn(K, generator=torch.Generator().manual_seed(3), dtype=torch.float32).to(dev)
    buf = torch.zeros(s.numel() + 1, dtype=torch.float32, device=dev)
    s_off = buf[1:].view(M, K // 128)
    s_off.copy_(sd)
    assert s_off.data_ptr() % 16 == 4
    assert torch.equal(mq.int4_gemv(x, qd, s_off), mq.int4_gemv(x, qd, sd))


@pytest.mark.parametrize("fmt", ["fp8", "int4"])
@pytest.mark.parametrize("shape,n,reps", [((1024, 2048), 3, 7), ((4096, 1024), 2, 5), ((37, 128), 2, 9)], ids=str)
def test_fmt_gemv_repeat_parity(mq, dev, fmt, shape, n, reps):
    M, K = shape
    print(f"{fmt} gemv repeat {M}x{K} copies={n} reps={reps}", flush=True)
    quant = of.quantize_fp8_rows if fmt == "fp8" else of.quantize_int4_groups
    deq = of.dequant_fp8 if fmt == "fp8" else of.dequant_int4
    qs = [quant(_weights(M, K, seed=100 + c + M))[0] for c in range(n)]
    s = quant(_weights(M, K, seed=99))[1]                 # one scale array for every copy
    x = torch.randn(K, generator=torch.Generator().manual_seed(5), dtype=torch.float32)
    fn = mq.fp8_gemv_repeat if fmt == "fp8" else mq.int4_gemv_repeat
    y = fn(x.to(dev), torch.stack(qs).to(dev), s.to(dev), reps)
    torch.cuda.synchronize()
    got = y.cpu().double().numpy()
    for c in range(n):
        assert _rel(got[c], of.matvec_f64(deq(qs[c], s), x)) <= 1e-5, c
