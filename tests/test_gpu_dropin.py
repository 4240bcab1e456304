"""The drop-in from C: tests/native/dropin.c, a C99 program that includes
only include/pz_sampling_compat.h and links -lpzsample, the way the
reference's build would link the library in place of src/sampling.

  kat       the properties the reference's sampler tests check
            (tests/test_sampling.c:24-245), restated in the program.
  dispatch  the sampling block of generate.c:145-169 (plus sample_top_k) on
            seeded rows: every id and every final RNG state must equal the
            oracle's (orc_sample_step with the row's own seeded state).

The program runs as a child process of the test."""
import os
import struct
import subprocess
import tempfile

import numpy as np
import pytest

import pz_oracle as po

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "dropin")


def test_dropin_known_answers():
    print("case dropin kat", flush=True)
    r = subprocess.run([BIN, "kat"], capture_output=True, text=True, timeout=120)
    print(r.stdout.strip(), flush=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_dropin_generate_dispatch_matches_oracle():
    rng = np.random.default_rng(0xD0)
    V = 32000
    cases = [(0.0, 1.0, 0), (0.8, 0.9, 0), (0.7, 0.95, 0), (1.0, 1.0, 0), (0.9, 0.0, 0),
             (0.8, 1.0, 40), (1.2, 1.0, 1), (0.5, 0.5, 0), (1e-7, 0.9, 0), (2.0, 1.0, 0)]
    rows = []
    for i in range(40):
        T, p, k = cases[i % len(cases)]
        rows.append((T, p, k, int(rng.integers(0, 2**63)) if i % 7 else 0))
    x = (rng.standard_normal((len(rows), V)) * 2.5).astype(np.float32)
    x[3, 0] = np.nan   # a NaN first logit on a top-p row
    with tempfile.TemporaryDirectory() as d:
        fin, fout = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        with open(fin, "wb") as f:
            f.write(struct.pack("<ii", len(rows), V))
            for T, p, k, seed in rows:
                f.write(struct.pack("<ffiQ", T, p, k, seed))
            f.write(x.tobytes())
        print("case dropin dispatch", flush=True)
        r = subprocess.run([BIN, "dispatch", fin, fout], capture_output=True, text=True,
                           timeout=300)
        assert r.returncode == 0, r.stdout + r.stderr
        raw = open(fout, "rb").read()
    got = [struct.unpack_from("<iQ", raw, 12 * i) for i in range(len(rows))]
    o = po.oracle()
    for i, (T, p, k, seed) in enumerate(rows):
        st = np.zeros(1, np.uint64)
        s = po.ctypes.c_ulonglong()
        o.orc_rng_seed(po.ctypes.byref(s), seed)
        st[0] = s.value
        ids, _, _ = po.sample_step(x[i:i + 1], [po.params(temperature=T, top_k=k, top_p=p)], st)
        assert got[i] == (int(ids[0]), int(st[0])), (i, T, p, k, got[i], ids[0], st[0])
