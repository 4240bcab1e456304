"""Writes the golden fixtures of the sampling path from the REFERENCE sampler.

The reference's own C sources (src/sampling/*.c and src/math/softmax.c of
Project Zero) are compiled where they lie by oracle/Makefile into
oracle/_ref/libpzref_{avx512,avx2}.so; this script calls those binaries on
seeded synthetic inputs and stores the outputs.  Inputs are NOT stored: each
case names the libpzsynth generator and seeds that rebuild them bit-exactly.

    make -C oracle && python tests/golden/make_golden.py

Outputs (JSON, small): rng.json, argmax.json, temperature.json, softmax.json,
top_k.json, top_p.json.
"""
import ctypes
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "project-zero_amd"), os.path.join(ROOT, "oracle")]

import pz_oracle as po  # noqa: E402
import pzsample as pz  # noqa: E402

_P = ctypes.c_void_p


def f32bits(v):
    return int(np.float32(v).view(np.uint32))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def state(r, seed):
    s = ctypes.c_ulonglong()
    r.rng_seed(ctypes.byref(s), seed)
    return s


def gen_rows(kind, rows, V, seed, **kw):
    """Rebuilds the input rows a fixture case names."""
    if kind == "normal":
        x = pz.synth_normal(rows, V, kw["sigma"], seed)
    elif kind == "normal_spikes":
        x = pz.synth_normal(rows, V, kw["sigma"], seed)
        pz.synth_spikes(x, kw["spikes"], kw["lo"], kw["hi"], seed + 1)
    elif kind == "gumbel":
        x = pz.synth_gumbel(rows, V, kw["scale"], seed)
    elif kind == "quantized":  # many exact ties: normal rounded to 1/4
        x = np.round(pz.synth_normal(rows, V, kw["sigma"], seed) * 4.0) / 4.0
        x = x.astype(np.float32)
    else:
        raise ValueError(kind)
    return np.ascontiguousarray(x, np.float32)


def main():
    r512 = po.ref(True)
    r2 = po.ref(False)
    if r512 is None or r2 is None:
        sys.exit("oracle/_ref not built: run make -C oracle with the reference present")
    out = {}

    # rng (rng.c): first 256 draws and final state for several seeds
    rng = []
    for seed in [0, 1, 42, 12345, 111, 222, 0xFFFFFFFFFFFFFFFF, 0x9E3779B97F4A7C15]:
        s = state(r512, seed)
        draws = [f32bits(r512.rng_float(ctypes.byref(s))) for _ in range(256)]
        rng.append({"seed": seed, "draws_f32bits": draws, "state_after": s.value})
    out["rng"] = rng

    # argmax (argmax.c), including rows with many ties and a NaN at index 0
    cases = []
    for kind, V, kw in [("normal", 4096, {"sigma": 3.0}), ("quantized", 4096, {"sigma": 1.0}),
                        ("normal", 128256, {"sigma": 3.0})]:
        x = gen_rows(kind, 8, V, 0xA0 + V, **kw)
        ids = [int(r512.sample_argmax(x[i].ctypes.data_as(_P), V)) for i in range(8)]
        cases.append({"kind": kind, "rows": 8, "V": V, "seed": 0xA0 + V, "kw": kw, "ids": ids})
    out["argmax"] = cases

    # temperature (temperature.c) both builds: sha256 of the scaled rows
    temps = []
    for T in [0.7, 0.8, 1.0, 1.3, 2.0, 1e-7]:
        x = gen_rows("normal", 4, 49152, 0xB0, sigma=3.0)
        for form, lib in (("mul_recip", r512), ("div", r2)):
            y = x.copy()
            for i in range(4):
                lib.apply_temperature(y[i].ctypes.data_as(_P), 49152, ctypes.c_float(T))
            temps.append({"T": T, "form": form, "seed": 0xB0, "rows": 4, "V": 49152,
                          "sha256": sha(y)})
    out["temperature"] = temps

    # softmax (softmax.c): sha256 of outputs + a few probabilities
    sm = []
    for V, sigma in [(1000, 1.0), (49152, 3.0), (128256, 2.0)]:
        x = gen_rows("normal", 4, V, 0xC0 + V, sigma=sigma)
        y = x.copy()
        for i in range(4):
            r512.softmax(y[i].ctypes.data_as(_P), V)
        sm.append({"V": V, "sigma": sigma, "seed": 0xC0 + V, "rows": 4, "sha256": sha(y),
                   "p0_f32bits": [f32bits(y[i, 0]) for i in range(4)]})
    out["softmax"] = sm

    # top_k (top_k.c): ids for rows x k x draw seeds
    tk = []
    for kind, V, kw in [("normal", 49152, {"sigma": 3.0}), ("quantized", 8192, {"sigma": 1.0}),
                        ("gumbel", 151936, {"scale": 2.5})]:
        x = gen_rows(kind, 6, V, 0xD0 + V, **kw)
        for k in [1, 2, 20, 40, 1024, 5000, 0, -3]:
            ids = []
            for i in range(6):
                s = state(r512, 1000 * (i + 1) + k)
                ids.append(int(r512.sample_top_k(x[i].copy().ctypes.data_as(_P), V, k,
                                                 ctypes.byref(s))))
            tk.append({"kind": kind, "V": V, "kw": kw, "seed": 0xD0 + V, "rows": 6, "k": k,
                       "draw_seed_base": 1000, "ids": ids})
    out["top_k"] = tk

    # top_p (top_p.c) after apply_temperature (the generate.c:154-156 order)
    tp = []
    for kind, V, kw, T in [("normal_spikes", 128256, {"sigma": 2.0, "spikes": 5, "lo": 8.0,
                                                       "hi": 12.0}, 0.7),
                           ("normal", 49152, {"sigma": 3.0}, 0.8),
                           ("quantized", 8192, {"sigma": 1.0}, 1.0),
                           ("normal", 250000, {"sigma": 1.0}, 1.0)]:
        x = gen_rows(kind, 8, V, 0xE0 + V, **kw)
        for p in [0.5, 0.9, 0.95, 0.999]:
            ids = []
            for i in range(8):
                y = x[i].copy()
                r512.apply_temperature(y.ctypes.data_as(_P), V, ctypes.c_float(T))
                s = state(r512, 2000 * (i + 1) + int(p * 1000))
                ids.append(int(r512.sample_top_p(y.ctypes.data_as(_P), V, ctypes.c_float(p),
                                                 ctypes.byref(s))))
            tp.append({"kind": kind, "V": V, "kw": kw, "T": T, "seed": 0xE0 + V, "rows": 8,
                       "top_p": p, "draw_seed_base": 2000, "ids": ids})
    out["top_p"] = tp

    for name, data in out.items():
        with open(os.path.join(HERE, f"{name}.json"), "w") as f:
            json.dump(data, f, indent=1 if name != "rng" else None)
    print("wrote", ", ".join(f"{k}.json" for k in out))


if __name__ == "__main__":
    main()
