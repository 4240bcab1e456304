"""pz_spec_decode: the speculative decode loop around the device
verification with caller-supplied models and KV rollback, against the
oracle's restatement of the same loop (pz_oracle.spec_decode) over 24
rounds.  The toy models (tests/native/toy_model.hip, restated in numpy
below) derive every logit from a hash of the whole cached prefix and check
each forward's position against their cache length, so a missing or wrong
rollback changes the emitted tokens or counts a cache error."""
import ctypes
import os

import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
from conftest import to_dev

pytestmark = pytest.mark.gpu

TOY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "libpztoy.so")
K1 = 0x9E3779B97F4A7C15
K2 = 0xD1B54A32D192ED03
M64 = (1 << 64) - 1


def mix64(z):
    z = np.asarray(z, np.uint64)
    z = z ^ (z >> np.uint64(33))
    z = z * np.uint64(0xff51afd7ed558ccd)
    z = z ^ (z >> np.uint64(33))
    z = z * np.uint64(0xc4ceb9fe1a85ec53)
    return z ^ (z >> np.uint64(33))


class ToyNumpy:
    """The numpy restatement of toy_model.hip."""

    def __init__(self, B, V, max_len, seed, tokens, lens):
        self.V = V
        self.h = [np.zeros((B, max_len + 1), np.uint64) for _ in range(2)]
        self.len = [np.zeros(B, np.int64) for _ in range(2)]
        with np.errstate(over="ignore"):
            for m in range(2):
                for b in range(B):
                    self.h[m][b, 0] = np.uint64(seed ^ b)
                    for p in range(lens[b] - 1):
                        self.h[m][b, p + 1] = mix64(self.h[m][b, p] ^ np.uint64(
                            ((int(tokens[b, p]) + 1) * K1) & M64))
                    self.len[m][b] = lens[b] - 1
        v1 = (np.arange(V, dtype=np.uint64) + np.uint64(1))
        with np.errstate(over="ignore"):
            self.vk1 = v1 * np.uint64(K1)
            self.vk2 = v1 * np.uint64(K2)

    def _rows(self, seeds, target):
        with np.errstate(over="ignore"):
            b24 = (mix64(seeds[:, None] ^ self.vk1[None, :]) >> np.uint64(40)).astype(np.int64)
            x = ((b24 - (1 << 23)).astype(np.float32) * np.float32(2.0 ** -21))
            if target:
                p21 = (mix64(seeds[:, None] ^ self.vk2[None, :]) >> np.uint64(43)).astype(np.int64)
                x = x + (p21 - (1 << 20)).astype(np.float32) * np.float32(2.0 ** -21)
        return x.astype(np.float32)

    def _advance(self, m, tok, pos):
        B, n = tok.shape
        seeds = np.empty((B, n), np.uint64)
        with np.errstate(over="ignore"):
            for b in range(B):
                assert pos[b] == self.len[m][b]
                for j in range(n):
                    p = pos[b] + j
                    self.h[m][b, p + 1] = mix64(self.h[m][b, p] ^ np.uint64(
                        ((int(tok[b, j]) + 1) * K1) & M64))
                    seeds[b, j] = self.h[m][b, p + 1]
                self.len[m][b] = pos[b] + n
        return seeds

    def draft(self, tok, pos):
        s = self._advance(0, np.asarray(tok)[:, None], pos)
        return self._rows(s[:, 0], False)

    def target(self, tok, pos):
        s = self._advance(1, np.asarray(tok), pos)
        B, n = s.shape
        return self._rows(s.ravel(), True).reshape(B, n, self.V)

    def rollback(self, m, pos):
        assert (pos <= self.len[m]).all()
        self.len[m][:] = pos


class SpecOpts(ctypes.Structure):
    _fields_ = [("greedy_draft", ctypes.c_int), ("stop_at_eos", ctypes.c_int)]


class SpecModels(ctypes.Structure):
    _fields_ = [("ctx", ctypes.c_void_p), ("draft_step", ctypes.c_void_p),
                ("target_forward", ctypes.c_void_p), ("kv_rollback", ctypes.c_void_p)]


def run_case(torch, B, K, V, tau, rounds, seed, greedy=False, eos=None):
    max_len = 8 + rounds * (K + 1)
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, 8, B).astype(np.int32)
    tokens = np.zeros((B, max_len), np.int32)
    for b in range(B):
        tokens[b, :lens[b]] = rng.integers(0, V, lens[b])
    draft_seed = (np.arange(1, B + 1, dtype=np.uint64) * np.uint64(7919)) | np.uint64(1)
    verify_seed = (np.arange(1, B + 1, dtype=np.uint64) * np.uint64(104729)) ^ np.uint64(5)
    toy_seed = 0xA11CE ^ seed
    # oracle
    o_tokens, o_lens = tokens.copy(), lens.copy().astype(np.int64)
    o_ds, o_vs = draft_seed.copy(), verify_seed.copy()
    model = ToyNumpy(B, V, max_len, toy_seed, tokens, lens)
    o_done = np.zeros(B, np.uint8)
    want_acc = po.spec_decode(model, B, K, V, tau, o_tokens, o_lens, rounds, o_ds, o_vs,
                              greedy_draft=greedy, eos=eos, done=o_done)
    # device
    lib = ctypes.CDLL(TOY)
    lib.toy_create.restype = ctypes.c_void_p
    lib.toy_create.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                               ctypes.c_void_p, ctypes.c_void_p]
    lib.toy_destroy.argtypes = [ctypes.c_void_p]
    lib.toy_errors.argtypes = [ctypes.c_void_p]
    g_tokens, g_lens = tokens.copy(), lens.copy()
    ctx = lib.toy_create(B, V, max_len, toy_seed, g_tokens.ctypes.data, g_lens.ctypes.data)
    assert ctx
    m = SpecModels(ctx, ctypes.cast(lib.toy_draft_step, ctypes.c_void_p).value,
                   ctypes.cast(lib.toy_target_forward, ctypes.c_void_p).value,
                   ctypes.cast(lib.toy_kv_rollback, ctypes.c_void_p).value)
    d_ds = to_dev(torch, draft_seed.view(np.int64))
    g_vs = verify_seed.copy()
    acc = np.zeros((rounds, B), np.int32)
    done = np.zeros(B, np.uint8)
    with pz.Sampler(B, V) as s:
        assert s.lib.pz_spec_decode.argtypes is not None
        torch.cuda.synchronize()
        if greedy or eos is not None:
            if eos is not None:
                s.set_eos(eos)
            opts = SpecOpts(int(greedy), int(eos is not None))
            rc = s.lib.pz_spec_decode_opts(s.h, ctypes.addressof(m), ctypes.addressof(opts), B,
                                           K, V, tau, g_tokens.ctypes.data, g_lens.ctypes.data,
                                           max_len, rounds, d_ds.data_ptr(), g_vs.ctypes.data,
                                           acc.ctypes.data, done.ctypes.data)
        else:
            rc = s.lib.pz_spec_decode(s.h, ctypes.addressof(m), B, K, V, tau,
                                      g_tokens.ctypes.data, g_lens.ctypes.data, max_len, rounds,
                                      d_ds.data_ptr(), g_vs.ctypes.data, acc.ctypes.data)
        assert rc == pz.PZ_OK, s.lib.pz_sampler_last_error(s.h)
    errors = lib.toy_errors(ctx)
    lib.toy_destroy(ctx)
    assert errors == 0, f"{errors} cache errors"
    print(f"B={B} K={K} V={V} tau={tau}: {rounds} rounds, accepted per round "
          f"{acc.mean():.2f} (min {acc.min()}, max {acc.max()}), "
          f"{int((acc == K).sum())} all-accepted, {int((acc == 0).sum())} immediate rejections",
          flush=True)
    assert (acc == want_acc).all()
    assert (g_lens == o_lens).all()
    assert (g_tokens == o_tokens).all()
    assert (g_vs == o_vs).all()
    assert (d_ds.cpu().numpy().view(np.uint64) == o_ds).all()
    assert (done == o_done).all()
    return acc, done


@pytest.mark.parametrize("B,K,V,tau", [(4, 4, 4096, 0.8), (3, 7, 1000, 1.3), (1, 1, 257, 0.5)])
def test_spec_decode_loop_matches_oracle(torch_cuda, B, K, V, tau):
    print(f"case specdec B={B} K={K} V={V} tau={tau}", flush=True)
    acc, _ = run_case(torch_cuda, B, K, V, tau, rounds=24, seed=B * 100 + K)
    # the trace exercises acceptances and rejections
    assert acc.max() >= 1 and acc.min() < K


@pytest.mark.parametrize("B,K,V,tau", [(4, 4, 64, 0.3), (3, 5, 257, 0.5)])
def test_spec_decode_greedy_drafts(torch_cuda, B, K, V, tau):
    """Greedy drafting: argmax drafts (no draws: the draft RNG states stay)
    verified with q one-hot."""
    print(f"case specdec greedy B={B} K={K} V={V} tau={tau}", flush=True)
    acc, _ = run_case(torch_cuda, B, K, V, tau, rounds=24, seed=B * 100 + K + 7, greedy=True)
    assert acc.max() >= 1


@pytest.mark.parametrize("greedy", [False, True])
def test_spec_decode_stops_at_eos(torch_cuda, greedy):
    """EOS ids end sequences (not committed); stopped sequences keep their
    tokens, states and caches through the remaining rounds."""
    B, K, V, tau = 6, 3, 1000, 0.9
    eos = list(range(7, V, 41))  # 24 ids
    print(f"case specdec eos greedy={greedy} B={B} K={K} V={V}", flush=True)
    acc, done = run_case(torch_cuda, B, K, V, tau, rounds=24, seed=4242 + int(greedy),
                         greedy=greedy, eos=eos)
    assert done.any(), "no sequence reached an EOS id"
    for b in np.nonzero(done)[0]:  # once stopped, a sequence takes no part
        stopped = np.nonzero(acc[:, b] < 0)[0]
        if stopped.size:
            assert (acc[stopped[0]:, b] < 0).all()
