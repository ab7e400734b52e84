"""kvt_decode_combine through the C ABI against a float64 merge of the same partials.

The split merge is out[b, hq, :] = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c over the splits in use of (b, KV
head hq / gs): partials carry m in natural-log units, o unnormalized, l the weight sum (the split-K kernels' layout:
slot (b * H + h) * n_chunks + c, q head j of the group at row slot * gs + j).  The cases cover one round of up to 256
splits and several rounds, empty splits (m = -inf, o = 0, l = 0), slots past the splits in use filled with NaN (they
must be selected out, not scaled by zero), a sequence with no split at all (0/0 = NaN, as the reference's chunk kernel,
gemv/test_kv_paged_prefix.py:524-526), the chunk > 0 mode (splits in use from the sequence length) and bf16 output
(the fp32 result rounded to nearest even), at split counts that give the kernel one to four wavefronts per block
and, with one wavefront, each of its 1 to 8 loads per lane.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

H, GS, D = 2, 8, 256
HQ = H * GS


def _partials(batch: int, n_chunks: int, used, seed: int):
    """Random partials: maxima spread over +-20 (natural log units), o and l of the size a split of a few hundred
    positions gives; every fifth split in use empty; NaN in every slot past `used`."""
    g = np.random.default_rng(seed)
    rows = batch * H * n_chunks * GS
    o = g.standard_normal((rows, D)) * 40.0
    m = g.uniform(-20.0, 20.0, rows)
    l = g.uniform(0.5, 300.0, rows)
    slot = np.arange(rows) // GS
    c = slot % n_chunks
    b = slot // (H * n_chunks)
    use = np.array([c[i] < used[b[i]] for i in range(rows)])
    empty = use & (c % 5 == 3)
    m[empty], l[empty], o[empty] = -np.inf, 0.0, 0.0
    m[~use], l[~use], o[~use] = np.nan, np.nan, np.nan
    return o.astype(np.float32), np.stack([m, l], 1).astype(np.float32), use


def _merge64(o, ml, use, batch, n_chunks):
    out = np.full((batch, HQ, D), np.nan)
    o = o.astype(np.float64).reshape(batch, H, n_chunks, GS, D)
    m = ml[:, 0].astype(np.float64).reshape(batch, H, n_chunks, GS)
    l = ml[:, 1].astype(np.float64).reshape(batch, H, n_chunks, GS)
    u = use.reshape(batch, H, n_chunks, GS)
    for b in range(batch):
        for h in range(H):
            for j in range(GS):
                sel = u[b, h, :, j] & np.isfinite(m[b, h, :, j])
                if not sel.any():
                    continue
                mm = m[b, h, sel, j]
                w = np.exp(mm - mm.max())
                out[b, h * GS + j] = (w[:, None] * o[b, h, sel, j]).sum(0) / (w * l[b, h, sel, j]).sum()
    return out


def _combine(o, ml, batch, n_chunks, chunk, seq_lens, counts, out_dtype):
    from kvtier import _lib
    dev = "cuda:0"
    po = torch.from_numpy(o).to(dev)
    pml = torch.from_numpy(ml).to(dev)
    sl = torch.tensor(seq_lens, dtype=torch.int32, device=dev)
    sc = None if counts is None else torch.tensor(counts, dtype=torch.int32, device=dev)
    out = torch.empty(batch, HQ, D, dtype=out_dtype, device=dev)
    _lib.call("kvt_decode_combine", po.data_ptr(), pml.data_ptr(), batch, H, HQ, D, n_chunks, chunk, sl.data_ptr(),
              _lib.ptr(sc), out.data_ptr() if out_dtype == torch.float32 else None,
              out.data_ptr() if out_dtype == torch.bfloat16 else None, out.stride(0), _lib.stream())
    torch.cuda.synchronize()
    return out.cpu()


def _check(got, want):
    nan_w = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan_w), "NaN pattern differs from the float64 merge"
    g, w = got[~nan_w], want[~nan_w]
    err = np.abs(g - w)
    assert float((err / (np.abs(w) + 1.0)).max()) < 2e-5, float(err.max())


@pytest.mark.parametrize("n_chunks", [1, 9, 17, 25, 33, 41, 49, 57, 64, 65, 100, 150, 192, 256, 257, 600])
def test_combine_split_counts(kvt_pkg, n_chunks):
    """chunk = 0: sequence b uses its first split_counts[b] slots (all, about half, none)."""
    batch = 3
    used = [n_chunks, max(1, n_chunks // 2), 0]
    o, ml, use = _partials(batch, n_chunks, used, seed=n_chunks)
    got = _combine(o, ml, batch, n_chunks, 0, [1, 1, 1], used, torch.float32).numpy().astype(np.float64)
    _check(got, _merge64(o, ml, use, batch, n_chunks))
    assert np.isnan(got[2]).all()


@pytest.mark.parametrize("n_chunks,chunk,lens", [(300, 64, [19_137, 64 * 300, 1]), (40, 512, [20_000, 700, 0])])
def test_combine_chunk_mode(kvt_pkg, n_chunks, chunk, lens):
    """chunk > 0: sequence b uses splits c < ceil(len_b / chunk) (at most n_chunks)."""
    batch = len(lens)
    used = [min(n_chunks, -(-L // chunk)) for L in lens]
    o, ml, use = _partials(batch, n_chunks, used, seed=chunk)
    got = _combine(o, ml, batch, n_chunks, chunk, lens, None, torch.float32).numpy().astype(np.float64)
    _check(got, _merge64(o, ml, use, batch, n_chunks))


@pytest.mark.parametrize("n_chunks", [40, 300])
def test_combine_bf16_is_rounded_fp32(kvt_pkg, n_chunks):
    """bf16 output = the fp32 output rounded to nearest even, bit for bit (NaN rows included); one wavefront per
    block (40 splits) and four (300)."""
    batch = 2
    used = [n_chunks, 0]
    o, ml, _ = _partials(batch, n_chunks, used, seed=7)
    f32 = _combine(o, ml, batch, n_chunks, 0, [1, 1], used, torch.float32)
    b16 = _combine(o, ml, batch, n_chunks, 0, [1, 1], used, torch.bfloat16)
    want = f32.to(torch.bfloat16)
    assert torch.equal(b16[0].view(torch.int16), want[0].view(torch.int16))
    assert bool(torch.isnan(b16[1].float()).all())
