"""Synthetic workloads of the sampling path (host arrays, seeded).

Each builder returns a dict with the host inputs of one configuration:
  logits [B, V] float32, params (list of pzsample.RowParams), u [B] uniforms,
  hist [B, H] int32 or None, and the algorithmic HBM bytes of one batch
  (one compulsory read of every logits row + side inputs + output ids).

  c1  single sequence, V=49152, N(0,3^2); repetition 1.1 over 64 ids, T 0.8,
      top-k 40, top-p 0.95, one draw per step (steps = rows here)
  c2  64 x 128256, N(0,2^2) + 5 spikes/row of +U[8,12]; T 0.7, top-p 0.9
  c3  256 x 151936, 2.5*Gumbel; presence 0.5 / frequency 0.3 from 512
      Zipf(1.1) ids; T 1.0, top-k 20, top-p 0.8
  c4  1024 x 128256, N(0,3^2); repetition 1.15 over 256 uniform ids; greedy
  c5  speculative verify: 32 seqs x 4 drafts x 128256, target N(0,2.5^2),
      draft = target + N(0,0.5^2), tau 0.8 (see build_c5)
  cat the plain path's full-vocabulary draw (the HTTP default T 1.0, top-p
      1.0: softmax + ascending-id CDF, generate.c:157-169) over c2's logits
"""
import numpy as np

import pzsample as pz

SEEDS = {"c1": 0xC1, "c2": 0xC2, "c3": 0xC3, "c4": 0xC4, "c5": 0xC5, "cat": 0xCA}


def _draw_seed(base):
    return base * 0x100000001 + 7


def build_c1(steps=500, V=49152, seed=None):
    seed = SEEDS["c1"] if seed is None else seed
    x = pz.synth_normal(steps, V, 3.0, seed)
    hist = pz.synth_uniform_ids(steps, 64, V, seed + 1)
    prm = pz.row_params(temperature=0.8, top_k=40, top_p=0.95, rep_penalty=1.1)
    u = pz.synth_draws(steps, _draw_seed(seed))
    return dict(name="c1", logits=x, params=[prm], u=u, hist=hist,
                bytes_per_row=V * 4 + 64 * 4 + 4)


def build_c2(B=64, V=128256, seed=None):
    seed = SEEDS["c2"] if seed is None else seed
    x = pz.synth_normal(B, V, 2.0, seed)
    pz.synth_spikes(x, 5, 8.0, 12.0, seed + 1)
    prm = pz.row_params(temperature=0.7, top_p=0.9)
    u = pz.synth_draws(B, _draw_seed(seed))
    # draw_seed: u[b] is rng_float of a state rng_seed(draw_seed ^ (b + 1))
    return dict(name="c2", logits=x, params=[prm], u=u, hist=None, draw_seed=_draw_seed(seed),
                bytes_per_row=V * 4 + 4 + 4)


def build_cat(B=64, V=128256, seed=None):
    seed = SEEDS["cat"] if seed is None else seed
    x = pz.synth_normal(B, V, 2.0, seed)
    pz.synth_spikes(x, 5, 8.0, 12.0, seed + 1)
    prm = pz.row_params(temperature=1.0)
    u = pz.synth_draws(B, _draw_seed(seed))
    return dict(name="cat", logits=x, params=[prm], u=u, hist=None,
                bytes_per_row=V * 4 + 4 + 4)


def build_c3(B=256, V=151936, H=512, seed=None):
    seed = SEEDS["c3"] if seed is None else seed
    x = pz.synth_gumbel(B, V, 2.5, seed)
    hist = pz.synth_zipf_ids(B, H, V, 1.1, seed + 1)
    prm = pz.row_params(temperature=1.0, top_k=20, top_p=0.8, presence_penalty=0.5,
                        frequency_penalty=0.3)
    u = pz.synth_draws(B, _draw_seed(seed))
    return dict(name="c3", logits=x, params=[prm], u=u, hist=hist,
                bytes_per_row=V * 4 + H * 4 + 4 + 4)


def build_c4(B=1024, V=128256, H=256, seed=None):
    seed = SEEDS["c4"] if seed is None else seed
    x = pz.synth_normal(B, V, 3.0, seed)
    hist = pz.synth_uniform_ids(B, H, V, seed + 1)
    prm = pz.row_params(temperature=0.0, rep_penalty=1.15)
    return dict(name="c4", logits=x, params=[prm], u=None, hist=hist,
                bytes_per_row=V * 4 + H * 4 + 4)


def build_c5(B=32, K=4, V=128256, has_bonus=True, seed=None):
    """Target rows [B, K+1, V] (row K is the bonus row), draft rows [B, K, V],
    draft ids sampled from q = softmax(draft/tau) on the host with the
    ascending-id categorical rule, acceptance uniforms [B, K], residual [B]."""
    seed = SEEDS["c5"] if seed is None else seed
    KT = K + (1 if has_bonus else 0)
    tau = 0.8
    target = pz.synth_normal(B * KT, V, 2.5, seed).reshape(B, KT, V)
    draft = pz.synth_perturb(np.ascontiguousarray(target[:, :K, :]).reshape(B * K, V), 0.5,
                             seed + 1).reshape(B, K, V)
    draft_ids = pz.synth_draft_ids(draft.reshape(B * K, V), tau, seed + 2).reshape(B, K)
    u_acc = pz.synth_draws(B * K, _draw_seed(seed)).reshape(B, K)
    u_res = pz.synth_draws(B, _draw_seed(seed) + 1)
    return dict(name="c5", target=target, draft=draft, draft_ids=draft_ids, u_acc=u_acc,
                u_res=u_res, B=B, K=K, V=V, has_bonus=has_bonus, tau=tau,
                bytes_per_seq=(2 * K + (1 if has_bonus else 0)) * V * 4 + K * 8 + 4 + (K + 2) * 4)


BUILDERS = {"c1": build_c1, "c2": build_c2, "c3": build_c3, "c4": build_c4, "c5": build_c5,
            "cat": build_cat}
