"""ctypes wrapper of the CPU oracle (libpzoracle.so) and of the reference
sampler compiled from its own sources (_ref/libpzref_*.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# PZ_ORACLE_LIB selects another build of the same source (bench.py's
# -march=native build on the timing host)
ORACLE_LIB = os.environ.get("PZ_ORACLE_LIB") or os.path.join(HERE, "libpzoracle.so")
REF_DIR = os.path.join(HERE, "_ref")

TEMP_MUL_RECIP, TEMP_DIV = 0, 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float
_ULL = ctypes.c_ulonglong
_pULL = ctypes.POINTER(ctypes.c_ulonglong)

PATH_ARGMAX, PATH_CATEGORICAL, PATH_TOPK, PATH_TOPP, PATH_CHAIN, PATH_TOPP_ARGMAX = range(6)


class OrcInfo(ctypes.Structure):
    _fields_ = [
        ("p_chosen", ctypes.c_float),
        ("dist_draw", ctypes.c_float),
        ("dist_cut", ctypes.c_float),
        ("cutoff", ctypes.c_int),
        ("n_cand", ctypes.c_int),
        ("trunc_sum", ctypes.c_float),
        ("norm_sum", ctypes.c_float),
        ("path", ctypes.c_int),
    ]


class OrcParams(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int),
        ("top_p", ctypes.c_float),
        ("rep_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
    ]


def params(temperature=1.0, top_k=0, top_p=1.0, rep_penalty=1.0,
           presence_penalty=0.0, frequency_penalty=0.0):
    return OrcParams(temperature, top_k, top_p, rep_penalty, presence_penalty,
                     frequency_penalty)


def _np(a):
    return a.ctypes.data_as(_P) if a is not None else None


_orc = None


def oracle():
    global _orc
    if _orc is not None:
        return _orc
    if not os.path.exists(ORACLE_LIB):
        raise RuntimeError(f"{ORACLE_LIB} missing: run make -C oracle")
    o = ctypes.CDLL(ORACLE_LIB)
    o.orc_rng_seed.argtypes = [_pULL, _ULL]
    o.orc_rng_seed.restype = None
    o.orc_rng_float.argtypes = [_pULL]
    o.orc_rng_float.restype = _F
    o.orc_argmax.argtypes = [_P, _I]
    o.orc_apply_temperature.argtypes = [_P, _I, _F, _I]
    o.orc_apply_temperature.restype = None
    o.orc_softmax.argtypes = [_P, _I]
    o.orc_softmax.restype = None
    o.orc_categorical.argtypes = [_P, _I, _F, ctypes.POINTER(OrcInfo)]
    o.orc_top_k.argtypes = [_P, _I, _I, _F, ctypes.POINTER(OrcInfo)]
    o.orc_top_p.argtypes = [_P, _I, _F, _F, ctypes.POINTER(OrcInfo)]
    o.orc_penalties.argtypes = [_P, _I, _P, _I, _F, _F, _F]
    o.orc_penalties.restype = None
    o.orc_chain.argtypes = [_P, _I, _I, _F, _F, ctypes.POINTER(OrcInfo)]
    o.orc_sample_row.argtypes = [_P, _I, ctypes.POINTER(OrcParams), _P, _I, _F, _I,
                                 ctypes.POINTER(OrcInfo)]
    o.orc_sample_batch.argtypes = [_P, _I, _I, _L, _P, _I, _P, _I, _P, _I, _P, _P, _P, _P]
    o.orc_sample_batch.restype = None
    o.orc_sample_step.argtypes = [_P, _I, _I, _L, _P, _I, _P, _I, _P, _I, _P, _I, _P, _P, _P]
    o.orc_sample_step.restype = None
    o.orc_spec_verify.argtypes = [_P, _P, _I, _I, _I, _I, _F, _I, _P, _P, _P, _P, _P, _P]
    o.orc_spec_verify.restype = None
    o.orc_expf.argtypes = [_F]
    o.orc_expf.restype = _F
    o.orc_expf_hash.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
    o.orc_expf_hash.restype = ctypes.c_uint64
    _orc = o
    return o


def sample_batch(x, params_list, u=None, hist=None, temp_mode=TEMP_MUL_RECIP):
    """Oracle over a [B, V] float32 array.  Returns ids, p_chosen, dist_draw, dist_cut."""
    x = np.ascontiguousarray(x, np.float32)
    B, V = x.shape
    if isinstance(params_list, OrcParams):
        params_list = [params_list]
    parr = (OrcParams * len(params_list))(*params_list)
    u = np.zeros(B, np.float32) if u is None else np.ascontiguousarray(u, np.float32)
    H = 0
    if hist is not None:
        hist = np.ascontiguousarray(hist, np.int32)
        H = hist.shape[1]
    ids = np.empty(B, np.int32)
    pc = np.empty(B, np.float32)
    dd = np.empty(B, np.float32)
    dc = np.empty(B, np.float32)
    oracle().orc_sample_batch(_np(x), B, V, V, parr, len(params_list), _np(hist), H, _np(u),
                              temp_mode, _np(ids), _np(pc), _np(dd), _np(dc))
    return ids, pc, dd, dc


def sample_step(x, params_list, state, hist=None, eos=(), temp_mode=TEMP_MUL_RECIP,
                workers=1):
    """One decode step over [B, V] with per-row RNG states (uint64[B],
    advanced in place).  Returns ids, EOS flags (uint8) and whether each row
    drew.  workers > 1 runs row blocks on that many threads (the oracle's
    work buffers are per thread; ctypes releases the GIL)."""
    x = np.ascontiguousarray(x, np.float32)
    B, V = x.shape
    if isinstance(params_list, OrcParams):
        params_list = [params_list]
    assert state.dtype == np.uint64 and state.flags.c_contiguous and state.size == B
    H = 0
    if hist is not None:
        hist = np.ascontiguousarray(hist, np.int32)
        H = hist.shape[1]
    eos = np.ascontiguousarray(eos, np.int32).ravel()
    ids = np.empty(B, np.int32)
    flags = np.empty(B, np.uint8)
    drew = np.empty(B, np.int32)
    o = oracle()

    def run(lo, hi):
        pl = params_list if len(params_list) == 1 else params_list[lo:hi]
        parr = (OrcParams * len(pl))(*pl)
        o.orc_sample_step(_np(x[lo:hi]), hi - lo, V, V, parr, len(pl),
                          _np(hist[lo:hi]) if hist is not None else None, H,
                          _np(state[lo:hi]), temp_mode, _np(eos) if eos.size else None,
                          int(eos.size), _np(ids[lo:hi]), _np(flags[lo:hi]), _np(drew[lo:hi]))

    if workers <= 1 or B < 2:
        run(0, B)
    else:
        from concurrent.futures import ThreadPoolExecutor
        n = min(workers, B)
        cuts = [B * i // n for i in range(n + 1)]
        with ThreadPoolExecutor(n) as ex:
            list(ex.map(lambda i: run(cuts[i], cuts[i + 1]), range(n)))
    return ids, flags, drew.astype(bool)


def sample_row(x, prm, u=0.0, hist=None, temp_mode=TEMP_MUL_RECIP):
    x = np.ascontiguousarray(x, np.float32)
    info = OrcInfo()
    H = 0
    if hist is not None:
        hist = np.ascontiguousarray(hist, np.int32)
        H = hist.shape[-1]
    rid = oracle().orc_sample_row(_np(x), x.shape[-1], ctypes.byref(prm), _np(hist), H,
                                  float(u), temp_mode, ctypes.byref(info))
    return rid, info


def spec_verify(target, draft, K, has_bonus, tau, draft_ids, u_acc, u_res,
                temp_mode=TEMP_MUL_RECIP):
    """draft None: greedy drafting, q one-hot at each draft id."""
    target = np.ascontiguousarray(target, np.float32)
    V = target.shape[-1]
    if draft is None:
        B = np.asarray(draft_ids).reshape(-1, K).shape[0]
    else:
        draft = np.ascontiguousarray(draft, np.float32)
        B = draft.shape[0] // K if draft.ndim == 2 else draft.shape[0]
    acc = np.empty(B, np.int32)
    out = np.empty((B, K + 1), np.int32)
    dist = np.empty(B, np.float32)
    oracle().orc_spec_verify(_np(target), _np(draft), B, K, V, int(has_bonus), tau, temp_mode,
                             _np(np.ascontiguousarray(draft_ids, np.int32)),
                             _np(np.ascontiguousarray(u_acc, np.float32)),
                             _np(np.ascontiguousarray(u_res, np.float32)),
                             _np(acc), _np(out), _np(dist))
    return acc, out, dist


# ---------------------------------------------------------------------------
# The reference sampler compiled from its sources (oracle/Makefile `ref`).
# ---------------------------------------------------------------------------
def host_has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            return " avx512f" in f.read()
    except OSError:
        return False


def ref_lib_path(avx512=None):
    if avx512 is None:
        avx512 = host_has_avx512()
    return os.path.join(REF_DIR, "libpzref_avx512.so" if avx512 else "libpzref_avx2.so")


_refs = {}


def ref(avx512=None):
    """The reference sampler (.so built from its own C sources), or None."""
    path = ref_lib_path(avx512)
    if path in _refs:
        return _refs[path]
    if not os.path.exists(path):
        return None
    r = ctypes.CDLL(path)
    r.rng_seed.argtypes = [_pULL, _ULL]
    r.rng_seed.restype = None
    r.rng_float.argtypes = [_pULL]
    r.rng_float.restype = _F
    r.sample_argmax.argtypes = [_P, _I]
    r.apply_temperature.argtypes = [_P, _I, _F]
    r.apply_temperature.restype = None
    r.sample_top_p.argtypes = [_P, _I, _F, _pULL]
    r.sample_top_k.argtypes = [_P, _I, _I, _pULL]
    r.softmax.argtypes = [_P, _I]
    r.softmax.restype = None
    _refs[path] = r
    return r


# ---------------------------------------------------------------------------
# The speculative decode loop (docs/architecture/IMPLEMENTATION_PLAN.md:
# 1675-1693, plan 18.2 / 18.3; not implemented in the reference): the round
# pz_spec_decode runs, restated over the oracle's own step and verification.
# ---------------------------------------------------------------------------
def spec_decode(models, B, K, V, tau, tokens, lens, rounds, draft_state, verify_state,
                temp_mode=TEMP_MUL_RECIP, greedy_draft=False, eos=None, done=None):
    """models: object with draft(tokens[B], pos[B]) -> [B, V] logits,
    target(tokens[B, n], pos[B]) -> [B, n, V] logits and rollback(model,
    pos[B]).  tokens [B, max_len] and lens [B] are advanced in place,
    draft_state (uint64 [B]) and verify_state (uint64 [B]) too.  Returns the
    accepted counts [rounds, B] (-1 for a sequence that had stopped).

    greedy_draft: each draft is the draft model's argmax (no draw; q is
    one-hot in the verification).  eos (ids) with done (uint8 [B], in/out):
    a sequence stops at the first committed id in eos, which is not
    committed (generate.c:198-211); from then on the sequence's tokens,
    length and RNG states stay as they are and both caches are rolled back
    to where they were."""
    o = oracle()
    acc_all = np.zeros((rounds, B), np.int32)
    q = np.empty((B, K, V), np.float32)
    prm = params(temperature=0.0 if greedy_draft else tau, top_k=0, top_p=1.0)
    eos = set(int(e) for e in (eos if eos is not None else ()))
    if done is None:
        done = np.zeros(B, np.uint8)
    for r in range(rounds):
        p0 = lens - 1
        x = tokens[np.arange(B), p0].copy()
        drafts = np.empty((B, K), np.int32)
        cur = x
        ds0 = draft_state.copy()
        for j in range(K + 1):
            lg = models.draft(cur, p0 + j)
            if j < K:
                q[:, j, :] = lg
                ids, _, _ = sample_step(lg, [prm], draft_state, temp_mode=temp_mode)
                drafts[:, j] = ids
                cur = ids
        draft_state[done != 0] = ds0[done != 0]  # a stopped sequence draws nothing
        tt = np.concatenate([x[:, None], drafts], axis=1)
        p = models.target(tt, p0)
        u_acc = np.zeros((B, K), np.float32)
        u_res = np.zeros(B, np.float32)
        for b in range(B):
            if done[b]:
                continue
            s = ctypes.c_ulonglong(int(verify_state[b]))
            for j in range(K):
                u_acc[b, j] = o.orc_rng_float(ctypes.byref(s))
            u_res[b] = o.orc_rng_float(ctypes.byref(s))
            verify_state[b] = s.value
        acc, out, _ = spec_verify(p, None if greedy_draft else q, K, True, tau, drafts, u_acc,
                                  u_res, temp_mode=temp_mode)
        pos_new = p0.copy()
        for b in range(B):
            if done[b]:
                acc_all[r, b] = -1
                continue
            a = int(acc[b])
            n = a + 1
            for i in range(a + 1):
                if int(out[b, i]) in eos:
                    n = i
                    done[b] = 1
                    break
            tokens[b, lens[b]:lens[b] + n] = out[b, :n]
            lens[b] += n
            pos_new[b] = p0[b] + n
            acc_all[r, b] = a
        models.rollback(0, pos_new)
        models.rollback(1, pos_new)
    return acc_all
