"""pz_sample_batch_noalloc (the allocation-free batched sampler, no sampler
object, scratch in one static device array per GPU) against the existing
pz_sample_batch_async on the same device inputs: ids and p(chosen) must be
bit-identical.  Two calls in a row, the second with a smaller input, then the
first again, so contents the array keeps from one call cannot leak into the
next; sizes beyond the stated maximum are rejected before anything runs.
The call also runs captured in a HIP graph (torch.cuda.CUDAGraph on a side
stream), replayed on new logits and uniforms in the same buffers: each
replay equals an eager call on the same inputs."""
import numpy as np
import pytest

import pzsample as pz
import workloads as wl
from conftest import to_dev

pytestmark = pytest.mark.gpu


def mixed_batch(B, V, seed):
    """Top-p rows (spiked N(0, 2^2), 0.7 / 0.9) with greedy, top-k chain,
    categorical and a flat row (every logit equal: more top-p candidates than
    the gather holds, so the fallback sort runs) mixed in."""
    x = pz.synth_normal(B, V, 2.0, seed)
    pz.synth_spikes(x, 5, 8.0, 12.0, seed + 1)
    x[3, :] = 0.25
    params = [pz.row_params(temperature=0.7, top_p=0.9) for _ in range(B)]
    params[1] = pz.row_params(temperature=0.0, rep_penalty=1.2)
    params[2] = pz.row_params(temperature=0.8, top_k=40, top_p=0.95, rep_penalty=1.1)
    params[3] = pz.row_params(temperature=0.7, top_p=0.9)
    if B > 5:
        params[5] = pz.row_params(temperature=0.9)
        params[B - 1] = pz.row_params(temperature=1.0, top_k=20, top_p=0.8,
                                      presence_penalty=0.5, frequency_penalty=0.3)
    return x, params


def run_pair(torch, x, params, u, hist, H):
    B, V = x.shape
    d_x = to_dev(torch, x)
    d_u = to_dev(torch, u[:B].astype(np.float32))
    d_h = to_dev(torch, hist) if H else None
    want_ids = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    want_p = torch.full((B,), -7.0, dtype=torch.float32, device="cuda")
    with pz.Sampler(B, V, max_hist=H) as s:
        torch.cuda.synchronize()
        s.sample_async(d_x, B, V, V, params, d_u, want_ids, want_p, d_hist=d_h, H=H)
        s.sync()
    got_ids = torch.full((B,), -9, dtype=torch.int32, device="cuda")
    got_p = torch.full((B,), -9.0, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = pz.sample_noalloc(d_x, B, V, V, params, d_u, got_ids, got_p, d_hist=d_h, H=H,
                           stream=stream)
    assert rc == pz.PZ_OK, rc
    torch.cuda.synchronize()
    gi, gp = got_ids.cpu().numpy(), got_p.cpu().numpy()
    wi, wp = want_ids.cpu().numpy(), want_p.cpu().numpy()
    assert (gi == wi).all(), (np.nonzero(gi != wi)[0][:8], gi[:8], wi[:8])
    assert (gp.view(np.uint32) == wp.view(np.uint32)).all(), np.nonzero(gp != wp)[0][:8]
    return gi


def test_noalloc_matches_async_twice_smaller_second(torch_cuda):
    H = 64
    # call 1: the configuration's full batch, 64 x 128256
    B1, V1 = 64, 128256
    print(f"case noalloc call1 B={B1} V={V1}", flush=True)
    x1, p1 = mixed_batch(B1, V1, 0x7A0)
    u1 = pz.synth_draws(B1, 0x7A1)
    h1 = pz.synth_uniform_ids(B1, H, V1, 0x7A2)
    first = run_pair(torch_cuda, x1, p1, u1, h1, H)
    # call 2: smaller batch and vocabulary, shared parameters (one mode)
    B2, V2 = 8, 49152
    print(f"case noalloc call2 B={B2} V={V2}", flush=True)
    x2 = pz.synth_normal(B2, V2, 3.0, 0x7A3)
    u2 = pz.synth_draws(B2, 0x7A4)
    h2 = pz.synth_uniform_ids(B2, H, V2, 0x7A5)
    run_pair(torch_cuda, x2, [pz.row_params(temperature=0.7, top_p=0.9)], u2, h2, H)
    # call 2b: smaller again, mixed modes
    B3, V3 = 6, 49152
    print(f"case noalloc call3 B={B3} V={V3}", flush=True)
    x3, p3 = mixed_batch(B3, V3, 0x7A6)
    run_pair(torch_cuda, x3, p3, pz.synth_draws(B3, 0x7A7),
             pz.synth_uniform_ids(B3, H, V3, 0x7A8), H)
    # call 1 again: identical to its first run
    print("case noalloc call1 again", flush=True)
    again = run_pair(torch_cuda, x1, p1, u1, h1, H)
    assert (again == first).all()


def test_noalloc_workload_c2(torch_cuda):
    """The top-p configuration as the bench draws it (64 x 128256, 0.7 / 0.9)."""
    w = wl.build_c2()
    print("case noalloc c2", flush=True)
    run_pair(torch_cuda, w["logits"], w["params"], w["u"], None, 0)


def test_noalloc_rejects_oversize(torch_cuda):
    d = torch_cuda.zeros((pz.PZ_NOALLOC_MAX_BATCH + 1, 16), dtype=torch_cuda.float32,
                         device="cuda")
    ids = torch_cuda.zeros((pz.PZ_NOALLOC_MAX_BATCH + 1,), dtype=torch_cuda.int32,
                           device="cuda")
    u = torch_cuda.zeros((pz.PZ_NOALLOC_MAX_BATCH + 1,), dtype=torch_cuda.float32,
                         device="cuda")
    prm = [pz.row_params(temperature=0.7, top_p=0.9)]
    assert pz.sample_noalloc(d, pz.PZ_NOALLOC_MAX_BATCH + 1, 16, 16, prm, u, ids) == pz.PZ_ERANGE
    # a vocabulary above the maximum (never read: rejected before any launch)
    assert pz.sample_noalloc(d, 1, pz.PZ_NOALLOC_MAX_VOCAB + 1, pz.PZ_NOALLOC_MAX_VOCAB + 1,
                             prm, u, ids) == pz.PZ_ERANGE
    assert pz.sample_noalloc(d, 1, 16, 16, prm, u, ids, d_hist=ids,
                             H=pz.PZ_NOALLOC_MAX_HIST + 1) == pz.PZ_ERANGE


def test_noalloc_graph_capture_replays(torch_cuda):
    torch = torch_cuda
    B, V, H = 16, 128256, 64
    x0 = pz.synth_normal(B, V, 2.0, 0x7C0)
    pz.synth_spikes(x0, 5, 8.0, 12.0, 0x7C1)
    params = [pz.row_params(temperature=0.7, top_p=0.9) for _ in range(B)]
    params[1] = pz.row_params(temperature=0.0, rep_penalty=1.2)
    params[2] = pz.row_params(temperature=0.8, top_k=40, top_p=0.95, rep_penalty=1.1)
    params[5] = pz.row_params(temperature=0.9)
    hist = pz.synth_uniform_ids(B, H, V, 0x7C2)
    d_x = to_dev(torch, x0)
    d_u = to_dev(torch, pz.synth_draws(B, 0x7C3).astype(np.float32))
    d_h = to_dev(torch, hist)
    ids = torch.full((B,), -9, dtype=torch.int32, device="cuda")
    p = torch.full((B,), -9.0, dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()
    # first call eagerly on the side stream (the per-device set-up runs here)
    with torch.cuda.stream(side):
        assert pz.sample_noalloc(d_x, B, V, V, params, d_u, ids, p, d_hist=d_h, H=H,
                                 stream=side.cuda_stream) == pz.PZ_OK
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("case noalloc capture B=16 V=128256", flush=True)
    with torch.cuda.graph(g, stream=side):
        rc = pz.sample_noalloc(d_x, B, V, V, params, d_u, ids, p, d_hist=d_h, H=H,
                               stream=side.cuda_stream)
    assert rc == pz.PZ_OK
    with pz.Sampler(B, V, max_hist=H) as s:
        want_ids = torch.full((B,), -7, dtype=torch.int32, device="cuda")
        want_p = torch.full((B,), -7.0, dtype=torch.float32, device="cuda")
        for k in range(3):
            print(f"case noalloc replay {k}", flush=True)
            xk = pz.synth_normal(B, V, 2.0, 0x7D0 + k)
            pz.synth_spikes(xk, 5, 8.0, 12.0, 0x7E0 + k)
            d_x.copy_(torch.from_numpy(xk))
            d_u.copy_(torch.from_numpy(pz.synth_draws(B, 0x7F0 + k).astype(np.float32)))
            ids.fill_(-9)
            p.fill_(-9.0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            # eager reference on the same inputs (between the replays)
            s.sample_async(d_x, B, V, V, params, d_u, want_ids, want_p, d_hist=d_h, H=H)
            s.sync()
            gi, gp = ids.cpu().numpy(), p.cpu().numpy()
            wi, wp = want_ids.cpu().numpy(), want_p.cpu().numpy()
            assert (gi == wi).all(), (k, np.nonzero(gi != wi)[0][:8], gi[:8], wi[:8])
            assert (gp.view(np.uint32) == wp.view(np.uint32)).all(), (k, np.nonzero(gp != wp)[0])
