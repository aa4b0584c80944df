"""Pins the W8A8 quantisation oracle with exact identities and brute force."""

from __future__ import annotations

import itertools

import torch

from oracle import quant_oracle as qo


def test_int8_accumulators_brute_force_and_identities():
    g = torch.Generator().manual_seed(7)
    a = torch.randint(-127, 128, (5, 256), generator=g, dtype=torch.int32).to(torch.int8)
    b = torch.randint(-127, 128, (3, 256), generator=g, dtype=torch.int32).to(torch.int8)
    acc = qo.int8_accumulate(a, b)
    for i, j in itertools.product(range(5), range(3)):
        assert int(acc[i, j]) == sum(int(x) * int(y) for x, y in zip(a[i].tolist(), b[j].tolist()))
    eye = torch.eye(256, dtype=torch.int8)
    assert torch.equal(qo.int8_accumulate(a, eye), a.to(torch.int32))
    assert torch.equal(qo.int8_accumulate(-a.to(torch.int32), b.to(torch.int32)), -acc)
    full = torch.full((1, 5120), 127, dtype=torch.int8)
    assert int(qo.int8_accumulate(full, full)) == 127 * 127 * 5120 < 2 ** 31


def test_int8_rows_round_half_even_and_zero_rows():
    x = torch.tensor([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -127.0, 3.49],
                      [0.0] * 8], dtype=torch.bfloat16)
    q, s = qo.int8_quantize_rows(x)
    assert s[0, 0].item() == 1.0
    assert s[1, 0].item() == torch.tensor(1e-12).item()
    assert q[0].tolist() == [127, 0, 2, 2, 0, -2, -127, 3]
    assert q[1].tolist() == [0] * 8


def test_fp8_codes_round_trip_saturate_and_ties():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    values = codes.view(torch.float8_e4m3fn).float()
    finite = torch.isfinite(values) & ~torch.isnan(values)
    back = values[finite].to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(back, codes[finite])
    # one row whose amax is 448 so the scale is exactly 1
    tiny = 2.0 ** -10   # half the smallest e4m3fn subnormal (2^-9)
    row = torch.tensor([[448.0, 1.0625, 1.1875, -tiny, tiny, 3 * tiny, 300.0]])
    q, s = qo.fp8_quantize_rows(row)
    assert s.item() == 1.0
    got = q.float()[0].tolist()
    assert got[0] == 448.0                 # largest finite e4m3fn
    assert got[1] == 1.0                   # 1.0625 is halfway between 1.0 and 1.125: even mantissa
    assert got[2] == 1.25                  # 1.1875 is halfway between 1.125 and 1.25: even mantissa
    assert got[3] == 0.0 and q.view(torch.uint8)[0, 3].item() == 0x80   # tie to zero keeps the sign
    assert got[4] == 0.0
    assert got[5] == 2 * 2.0 ** -9         # 1.5 subnormal steps: tie to the even step
    assert got[6] == 288.0                 # 300: nearest multiple of 32 above 256
    zero_q, zero_s = qo.fp8_quantize_rows(torch.zeros(2, 4))
    assert torch.all(zero_s == 1e-12) and torch.all(zero_q.float() == 0)
    big = torch.tensor([[1000.0, -1000.0]])
    assert qo.fp8_quantize_tensor(big)[0].float().abs().max().item() == 448.0
