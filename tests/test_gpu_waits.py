"""Bounded waits between the workgroups that share a row.

The host forces the give-up with a wait bound of one poll
(pz_sampler_set_wait_bound): every kernel still exits normally, each row's
id is either the oracle's or PZ_ID_FAILED, the synchronous call reports
PZ_EDEVICE when a row failed, and the next call with the default bound is
exact again (the failure path leaves the workspace clean)."""
import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
import workloads as wl
from conftest import to_dev

pytestmark = pytest.mark.gpu


def orc(p):
    return po.params(p.temperature, p.top_k, p.top_p, p.rep_penalty, p.presence_penalty,
                     p.frequency_penalty)


def forced(torch, w, tries=5):
    x, params, u, hist = w["logits"], w["params"], w["u"], w["hist"]
    B, V = x.shape
    H = hist.shape[1] if hist is not None else 0
    want, _, _, _ = po.sample_batch(x, [orc(q) for q in params], u=u, hist=hist)
    d_x = to_dev(torch, x)
    d_h = to_dev(torch, hist) if H else None
    d_u = to_dev(torch, (u if u is not None else np.zeros(B)).astype(np.float32))
    ids = torch.empty(B, dtype=torch.int32, device="cuda")
    failed = 0
    with pz.Sampler(B, V, max_hist=max(H, 1)) as s:
        s.set_wait_bound(1)
        for t in range(tries):
            print(f"case forced give-up {w['name']} B={B} try {t}", flush=True)
            ids.fill_(-9)
            s.sample_async(d_x, B, V, V, params, d_u, ids, d_hist=d_h, H=H)
            s.sync()
            got = ids.cpu().numpy()
            bad = got != want
            assert (got[bad] == pz.PZ_ID_FAILED).all(), (np.nonzero(bad)[0][:8], got[bad][:8])
            failed += int(bad.sum())
            if failed:
                break
        # the synchronous call reports a failed row as PZ_EDEVICE
        try:
            got, _ = s.sample(d_x, B, V, V, params, u=u, d_hist=d_h, H=H)
            assert (got == want).all()
        except pz.PzError as e:
            assert e.code == pz.PZ_EDEVICE, e
        # the default bound: exact on every row, twice
        s.set_wait_bound(0)
        for t in range(2):
            print(f"case default bound {w['name']} B={B} call {t}", flush=True)
            got, _ = s.sample(d_x, B, V, V, params, u=u, d_hist=d_h, H=H)
            assert (got == want).all(), np.nonzero(got != want)[0][:8]
    return failed


def test_top_p_front_waits_give_up_cleanly(torch_cuda):
    """C2 (64 x 128256): the front launch's meetings and histogram exchange."""
    failed = forced(torch_cuda, wl.build_c2())
    print(f"  rows that gave up: {failed}", flush=True)
    assert failed > 0  # one poll cannot see every slice of every row posted


def test_greedy_split_merge_bound(torch_cuda):
    """Greedy rows split over workgroups (8 x 128256): the last workgroup's
    reads of the others' posted words."""
    forced(torch_cuda, wl.build_c4(B=8))


def test_categorical_front_waits_give_up_cleanly(torch_cuda):
    """The categorical draw's front launch (64 x 128256): its two meetings."""
    failed = forced(torch_cuda, wl.build_cat())
    print(f"  rows that gave up: {failed}", flush=True)
    assert failed > 0
