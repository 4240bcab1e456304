"""Rows whose stride is a multiple of 4 while the vocabulary is not (50257
padded to 50304, the usual LM-head padding): the 128-bit load paths clamp
their last float4 to the row and the greedy kernel takes its scalar tail.
The padding holds huge values, so a kernel that read past V would pick them.
Ids and p(chosen) must be identical to the oracle on the first V columns."""
import ctypes

import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
from conftest import to_dev

pytestmark = pytest.mark.gpu

B, V, LD, H = 8, 50257, 50304, 64


def padded(seed):
    x = pz.synth_normal(B, V, 3.0, seed)
    full = np.full((B, LD), 1e30, np.float32)
    full[:, :V] = x
    return x, full


CASES = {
    "greedy": dict(temperature=0.0),
    "greedy_rep": dict(temperature=0.0, rep_penalty=1.3),
    "categorical": dict(temperature=0.9),
    "topk": dict(temperature=0.8, top_k=40),
    "chain": dict(temperature=0.8, top_k=50, top_p=0.9),
    "topp": dict(temperature=0.7, top_p=0.9),
    "topp_pres": dict(temperature=0.7, top_p=0.9, presence_penalty=0.5, frequency_penalty=0.3),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_padded_rows(torch_cuda, name):
    kw = CASES[name]
    print(f"case padded {name} B={B} V={V} ld={LD}", flush=True)
    x, full = padded(0x50 + len(name))
    hist = pz.synth_uniform_ids(B, H, V, 0x51)
    hist[:, 0] = V - 1  # the last real id
    u = pz.synth_draws(B, 0x52)
    d_x = to_dev(torch_cuda, full)
    d_h = to_dev(torch_cuda, hist)
    with pz.Sampler(B, V, max_hist=H) as s:
        ids, p = s.sample(d_x, B, V, LD, [pz.row_params(**kw)], u=u, d_hist=d_h, H=H,
                          want_p=True)
    want, wp, _, _ = po.sample_batch(x, [po.params(**kw)], u=u, hist=hist)
    assert (ids == want).all(), (name, ids, want)
    if not name.startswith("greedy"):
        assert (p.view(np.uint32) == wp.view(np.uint32)).all(), (name, p, wp)


def test_padded_softmax(torch_cuda):
    x, full = padded(0x60)
    d_in = to_dev(torch_cuda, full)
    d_out = torch_cuda.full((B, LD), -7.0, dtype=torch_cuda.float32, device="cuda")
    with pz.Sampler(B, V) as s:
        s.softmax(d_in, d_out, B, V, LD, LD, temperature=0.8)
        s.sync()
    got = d_out.cpu().numpy()
    want = x.copy()
    o = po.oracle()
    for b in range(B):
        row = want[b]
        o.orc_apply_temperature(row.ctypes.data_as(ctypes.c_void_p), V, ctypes.c_float(0.8), 0)
        o.orc_softmax(row.ctypes.data_as(ctypes.c_void_p), V)
    assert (got[:, :V].view(np.uint32) == want.view(np.uint32)).all()
    assert (got[:, V:] == -7.0).all()  # the padding of the output is not written
