"""ctypes binding of libpzsample.so (include/pz_sampler.h) and libpzsynth.so.

Host-side glue for tests and bench.py: the sampler itself is the HIP library;
this module only marshals arguments.  Device buffers may be given as integer
addresses or as torch tensors on the GPU (PyTorch is used for device memory
only).  Loading fails loudly when the library has not been built.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
SAMPLE_LIB = os.path.join(LIB_DIR, "libpzsample.so")
SYNTH_LIB = os.path.join(LIB_DIR, "libpzsynth.so")

PZ_OK, PZ_EINVAL, PZ_ENOMEM, PZ_EDEVICE, PZ_ERANGE, PZ_ENOTSUP = 0, -1, -2, -3, -4, -5
PZ_TEMP_MUL_RECIP, PZ_TEMP_DIV = 0, 1

# Every symbol include/pz_sampler.h and include/pz_sampling_compat.h declare.
ABI_SYMBOLS = (
    "pz_sampler_create", "pz_sampler_destroy", "pz_sampler_set_temp_mode",
    "pz_sampler_last_error", "pz_sampler_stream", "pz_sample_batch",
    "pz_sample_batch_async", "pz_sampler_sync", "pz_spec_verify", "pz_spec_verify_async",
    "pz_device_alloc", "pz_device_free", "pz_memcpy_h2d", "pz_memcpy_d2h",
    "pz_temperature_batch", "pz_softmax_batch", "pz_sample_batch_noalloc",
    "pz_sample_step", "pz_sampler_set_eos", "pz_attn_softmax", "pz_lm_head_bf16",
    "pz_lm_head_argmax_bf16", "pz_spec_decode", "pz_sampler_set_wait_bound",
    "pz_spec_verify_greedy", "pz_spec_verify_greedy_async", "pz_spec_decode_opts",
    # include/pz_sampling_compat.h: the reference sampler's own symbols
    "sample_argmax", "apply_temperature", "sample_top_p", "sample_top_k", "rng_seed",
    "rng_float", "pz_tn_softmax", "pz_compat_set_temp_mode", "pz_compat_last_status",
)


class PzError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"pz error {code}: {msg}")
        self.code = code


class RowParams(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("rep_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
    ]


def row_params(temperature=1.0, top_k=0, top_p=1.0, rep_penalty=1.0,
               presence_penalty=0.0, frequency_penalty=0.0):
    return RowParams(temperature, top_k, top_p, rep_penalty, presence_penalty,
                     frequency_penalty)


_lib = None
_synth = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float


def load():
    """Loads libpzsample.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(SAMPLE_LIB):
        raise RuntimeError(
            f"{SAMPLE_LIB} is missing: build the HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(SAMPLE_LIB)
    lib.pz_sampler_create.argtypes = [ctypes.POINTER(_P), _I, _I, _I, _I]
    lib.pz_sampler_destroy.argtypes = [_P]
    lib.pz_sampler_destroy.restype = None
    lib.pz_sampler_set_temp_mode.argtypes = [_P, _I]
    lib.pz_sampler_set_wait_bound.argtypes = [_P, ctypes.c_uint32]
    lib.pz_sampler_last_error.argtypes = [_P]
    lib.pz_sampler_last_error.restype = ctypes.c_char_p
    lib.pz_sampler_stream.argtypes = [_P]
    lib.pz_sampler_stream.restype = _P
    lib.pz_sample_batch.argtypes = [_P, _P, _I, _I, _L, _P, _I, _P, _I, _P, _P, _P]
    lib.pz_sample_batch_async.argtypes = [_P, _P, _I, _I, _L, _P, _I, _P, _I, _P, _P, _P]
    lib.pz_sampler_sync.argtypes = [_P]
    lib.pz_sample_step.argtypes = [_P, _P, _I, _I, _L, _P, _I, _P, _I, _P, _P, _P, _P]
    lib.pz_sampler_set_eos.argtypes = [_P, _P, _I]
    lib.pz_sample_batch_noalloc.argtypes = [_I, _P, _I, _P, _I, _I, _L, _P, _I, _P, _I, _P,
                                            _P, _P]
    lib.pz_spec_verify.argtypes = [_P, _P, _P, _I, _I, _I, _L, _I, _F, _P, _P, _P, _P, _P]
    lib.pz_spec_verify_async.argtypes = [_P, _P, _P, _I, _I, _I, _L, _I, _F, _P, _P, _P, _P,
                                         _P]
    lib.pz_device_alloc.argtypes = [ctypes.POINTER(_P), ctypes.c_size_t, _I]
    lib.pz_device_free.argtypes = [_P]
    lib.pz_memcpy_h2d.argtypes = [_P, _P, ctypes.c_size_t]
    lib.pz_memcpy_d2h.argtypes = [_P, _P, ctypes.c_size_t]
    lib.pz_temperature_batch.argtypes = [_P, _P, _L, _I, _I, _F]
    lib.pz_softmax_batch.argtypes = [_P, _P, _L, _P, _L, _I, _I, _F]
    lib.pz_attn_softmax.argtypes = [_P, _P, _L, _P, _L, _I, _I, _P]
    lib.pz_lm_head_bf16.argtypes = [_P, _P, _I, _I, _P, _I, _L, _P, _L]
    lib.pz_lm_head_argmax_bf16.argtypes = [_P, _P, _I, _I, _P, _I, _L, _P]
    lib.pz_spec_decode.argtypes = [_P, _P, _I, _I, _I, _F, _P, _P, _I, _I, _P, _P, _P]
    lib.pz_spec_decode_opts.argtypes = [_P, _P, _P, _I, _I, _I, _F, _P, _P, _I, _I, _P, _P, _P,
                                        _P]
    lib.pz_spec_verify_greedy.argtypes = [_P, _P, _I, _I, _I, _L, _I, _F, _P, _P, _P, _P, _P]
    lib.pz_spec_verify_greedy_async.argtypes = [_P, _P, _I, _I, _I, _L, _I, _F, _P, _P, _P,
                                                _P, _P]
    pull = ctypes.POINTER(ctypes.c_ulonglong)
    lib.sample_argmax.argtypes = [_P, _I]
    lib.apply_temperature.argtypes = [_P, _I, _F]
    lib.apply_temperature.restype = None
    lib.sample_top_p.argtypes = [_P, _I, _F, pull]
    lib.sample_top_k.argtypes = [_P, _I, _I, pull]
    lib.rng_seed.argtypes = [pull, ctypes.c_ulonglong]
    lib.rng_seed.restype = None
    lib.rng_float.argtypes = [pull]
    lib.rng_float.restype = _F
    lib.pz_tn_softmax.argtypes = [_P, _I]
    lib.pz_tn_softmax.restype = None
    lib.pz_compat_set_temp_mode.argtypes = [_I]
    lib.pz_compat_set_temp_mode.restype = None
    lib.pz_compat_last_status.argtypes = []
    _lib = lib
    return lib


def _ptr(x):
    """Device address of an int / torch tensor / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    raise TypeError(f"not a device buffer: {type(x)}")


def _np_ptr(a):
    return a.ctypes.data_as(_P) if a is not None else None


def _sync_torch(*bufs):
    for b in bufs:
        if hasattr(b, "is_cuda") and b.is_cuda:
            import torch
            torch.cuda.synchronize(b.device)
            return


def _params_array(params, B):
    if isinstance(params, RowParams):
        params = [params]
    params = list(params)
    if len(params) not in (1, B):
        raise ValueError("params must have 1 or B entries")
    arr = (RowParams * len(params))(*params)
    return arr, len(params)


class Sampler:
    """One pz_sampler (stream + scratch + staging) on one device."""

    def __init__(self, max_batch, max_vocab, max_hist=0, device=0,
                 temp_mode=PZ_TEMP_MUL_RECIP):
        self.lib = load()
        h = _P()
        rc = self.lib.pz_sampler_create(ctypes.byref(h), max_batch, max_vocab,
                                        max_hist, device)
        if rc != PZ_OK:
            raise PzError(rc, "pz_sampler_create failed")
        self.h = h
        self.set_temp_mode(temp_mode)

    def close(self):
        if self.h:
            self.lib.pz_sampler_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc):
        if rc != PZ_OK:
            raise PzError(rc, self.lib.pz_sampler_last_error(self.h).decode())

    def set_temp_mode(self, mode):
        self._check(self.lib.pz_sampler_set_temp_mode(self.h, mode))

    def set_wait_bound(self, polls):
        """Bound of the waits between a row's workgroups (0: the default)."""
        self._check(self.lib.pz_sampler_set_wait_bound(self.h, polls))

    @property
    def stream(self):
        return self.lib.pz_sampler_stream(self.h)

    def sample(self, d_logits, B, V, ld, params, u=None, d_hist=None, H=0,
               want_p=False):
        """Synchronous batched sampling; returns (ids int32[B], p float32[B]|None)."""
        _sync_torch(d_logits, d_hist)
        parr, n = _params_array(params, B)
        ids = np.empty(B, np.int32)
        p = np.empty(B, np.float32) if want_p else None
        ua = np.ascontiguousarray(u, np.float32).ravel() if u is not None else None
        if ua is not None and ua.size < B:
            raise ValueError(f"u holds {ua.size} uniforms, B={B} rows need {B}")
        rc = self.lib.pz_sample_batch(self.h, _ptr(d_logits), B, V, ld, parr, n,
                                      _ptr(d_hist), H, _np_ptr(ua), _np_ptr(ids),
                                      _np_ptr(p))
        self._check(rc)
        return ids, p

    def caller(self, B, V, ld, params, H=0):
        """A function f(d_logits, u, d_hist) -> ids for repeated synchronous
        calls of one shape: the arguments are marshalled once, so a call
        costs the library call itself (as a C caller pays), not the
        wrapper's per-call conversions.  d_logits / d_hist: device addresses
        (int); u: float32 array of B uniforms or None.  The returned ids
        array is reused by the next call."""
        parr, n = _params_array(params, B)
        ids = np.empty(B, np.int32)
        ub = np.empty(B, np.float32)
        pids, pu = _np_ptr(ids), _np_ptr(ub)
        f, h = self.lib.pz_sample_batch, self.h
        check = self._check

        def call(d_logits, u=None, d_hist=None):
            if u is not None:
                ub[:] = u
            rc = f(h, d_logits, B, V, ld, parr, n, d_hist, H, pu if u is not None else None,
                   pids, None)
            if rc:
                check(rc)
            return ids
        return call

    def sample_async(self, d_logits, B, V, ld, params, d_u, d_ids, d_p=None,
                     d_hist=None, H=0):
        parr, n = _params_array(params, B)
        rc = self.lib.pz_sample_batch_async(self.h, _ptr(d_logits), B, V, ld, parr, n,
                                            _ptr(d_hist), H, _ptr(d_u), _ptr(d_ids),
                                            _ptr(d_p))
        self._check(rc)

    def sync(self):
        self._check(self.lib.pz_sampler_sync(self.h))

    def set_eos(self, eos_ids):
        """EOS ids that sample_step flags (host list, copied)."""
        arr = np.ascontiguousarray(eos_ids, np.int32).ravel()
        self._check(self.lib.pz_sampler_set_eos(self.h, _np_ptr(arr), arr.size))

    def sample_step(self, d_logits, B, V, ld, params, d_state, d_ids, d_p=None, d_eos=None,
                    d_hist=None, H=0):
        """One decode step with device RNG states (u64[B]) and EOS flags
        (u8[B]); asynchronous on the sampler's stream."""
        parr, n = _params_array(params, B)
        rc = self.lib.pz_sample_step(self.h, _ptr(d_logits), B, V, ld, parr, n, _ptr(d_hist), H,
                                     _ptr(d_state), _ptr(d_ids), _ptr(d_p), _ptr(d_eos))
        self._check(rc)

    def temperature(self, d_x, B, V, ld, temperature):
        """In-place apply_temperature over device rows (asynchronous)."""
        _sync_torch(d_x)
        self._check(self.lib.pz_temperature_batch(self.h, _ptr(d_x), ld, B, V, temperature))

    def softmax(self, d_in, d_out, B, V, ld_in, ld_out, temperature=1.0):
        """Reference softmax of device rows into d_out (asynchronous)."""
        _sync_torch(d_in, d_out)
        self._check(self.lib.pz_softmax_batch(self.h, _ptr(d_in), ld_in, _ptr(d_out), ld_out, B,
                                              V, temperature))

    def attn_softmax(self, d_in, d_out, n_rows, n, ld_in, ld_out, d_len=None):
        """Reference softmax of attention-score rows, row r over its first
        min(d_len[r], n) entries (asynchronous)."""
        _sync_torch(d_in, d_out, d_len)
        self._check(self.lib.pz_attn_softmax(self.h, _ptr(d_in), ld_in, _ptr(d_out), ld_out,
                                             n_rows, n, _ptr(d_len)))

    def lm_head(self, d_w, V, n, d_x, B, ldx, d_logits, ld):
        """logits[b, i] = bf16 W[i, :] . x[b, :] (asynchronous)."""
        _sync_torch(d_w, d_x, d_logits)
        self._check(self.lib.pz_lm_head_bf16(self.h, _ptr(d_w), V, n, _ptr(d_x), B, ldx,
                                             _ptr(d_logits), ld))

    def lm_head_argmax(self, d_w, V, n, d_x, B, ldx, d_ids):
        """Greedy ids of the LM head's logits, argmax fused (asynchronous)."""
        _sync_torch(d_w, d_x, d_ids)
        self._check(self.lib.pz_lm_head_argmax_bf16(self.h, _ptr(d_w), V, n, _ptr(d_x), B, ldx,
                                                    _ptr(d_ids)))

    def spec_verify(self, d_target, d_draft, B, K, V, ld, has_bonus, temperature,
                    draft_ids, u_acc, u_res):
        """d_draft None: greedy drafts (pz_spec_verify_greedy, q one-hot)."""
        _sync_torch(d_target, d_draft)
        acc = np.empty(B, np.int32)
        out = np.empty((B, K + 1), np.int32)
        di = np.ascontiguousarray(draft_ids, np.int32).ravel()
        ua = np.ascontiguousarray(u_acc, np.float32).ravel()
        ur = np.ascontiguousarray(u_res, np.float32).ravel()
        for name, a, need in (("draft_ids", di, B * K), ("u_acc", ua, B * K), ("u_res", ur, B)):
            if a.size < need:
                raise ValueError(f"{name} holds {a.size} entries, B={B}, K={K} need {need}")
        if d_draft is None:
            rc = self.lib.pz_spec_verify_greedy(self.h, _ptr(d_target), B, K, V, ld,
                                                int(has_bonus), float(temperature), _np_ptr(di),
                                                _np_ptr(ua), _np_ptr(ur), _np_ptr(acc),
                                                _np_ptr(out))
        else:
            rc = self.lib.pz_spec_verify(self.h, _ptr(d_target), _ptr(d_draft), B, K, V, ld,
                                         int(has_bonus), float(temperature), _np_ptr(di),
                                         _np_ptr(ua), _np_ptr(ur), _np_ptr(acc), _np_ptr(out))
        self._check(rc)
        return acc, out

    def spec_verify_async(self, d_target, d_draft, B, K, V, ld, has_bonus, temperature,
                          d_draft_ids, d_u_acc, d_u_res, d_acc_len, d_ids_out):
        """pz_spec_verify_async: device inputs [B,K] int32 / [B,K] / [B] float32,
        device outputs [B] and [B,K+1] int32, enqueued on the sampler's stream."""
        _sync_torch(d_target, d_draft, d_draft_ids, d_u_acc, d_u_res, d_acc_len, d_ids_out)
        rc = self.lib.pz_spec_verify_async(self.h, _ptr(d_target), _ptr(d_draft), B, K, V, ld,
                                           int(has_bonus), float(temperature),
                                           _ptr(d_draft_ids), _ptr(d_u_acc), _ptr(d_u_res),
                                           _ptr(d_acc_len), _ptr(d_ids_out))
        self._check(rc)


# ---------------------------------------------------------------------------
# Synthetic workloads (libpzsynth.so)
# ---------------------------------------------------------------------------
def synth():
    global _synth
    if _synth is not None:
        return _synth
    if not os.path.exists(SYNTH_LIB):
        raise RuntimeError(f"{SYNTH_LIB} is missing: run the build first")
    s = ctypes.CDLL(SYNTH_LIB)
    u64 = ctypes.c_uint64
    d = ctypes.c_double
    s.pz_synth_normal.argtypes = [_P, _I, _I, _L, d, d, u64]
    s.pz_synth_gumbel.argtypes = [_P, _I, _I, _L, d, u64]
    s.pz_synth_spikes.argtypes = [_P, _I, _I, _L, _I, d, d, u64, _P]
    s.pz_synth_perturb.argtypes = [_P, _P, _I, _I, _L, d, u64]
    s.pz_synth_uniform_ids.argtypes = [_P, _I, _I, _I, u64]
    s.pz_synth_zipf_ids.argtypes = [_P, _I, _I, _I, d, u64]
    s.pz_synth_draws.argtypes = [_P, _I, u64]
    s.pz_synth_draft_ids.argtypes = [_P, _P, _I, _I, _L, _F, u64]
    _synth = s
    return s


def synth_normal(rows, V, sigma, seed, mean=0.0, ld=None):
    ld = ld or V
    out = np.zeros((rows, ld), np.float32)
    synth().pz_synth_normal(_np_ptr(out), rows, V, ld, mean, sigma, seed)
    return out


def synth_gumbel(rows, V, scale, seed):
    out = np.empty((rows, V), np.float32)
    synth().pz_synth_gumbel(_np_ptr(out), rows, V, V, scale, seed)
    return out


def synth_spikes(x, n_spikes, lo, hi, seed):
    rows, ld = x.shape
    ids = np.empty((rows, n_spikes), np.int32)
    synth().pz_synth_spikes(_np_ptr(x), rows, ld, ld, n_spikes, lo, hi, seed, _np_ptr(ids))
    return ids


def synth_perturb(x, sigma, seed):
    rows, V = x.shape
    out = np.empty_like(x)
    synth().pz_synth_perturb(_np_ptr(out), _np_ptr(x), rows, V, V, sigma, seed)
    return out


def synth_uniform_ids(rows, H, V, seed):
    out = np.empty((rows, H), np.int32)
    synth().pz_synth_uniform_ids(_np_ptr(out), rows, H, V, seed)
    return out


def synth_zipf_ids(rows, H, V, s, seed):
    out = np.empty((rows, H), np.int32)
    if synth().pz_synth_zipf_ids(_np_ptr(out), rows, H, V, s, seed) != 0:
        raise MemoryError("zipf table")
    return out


def synth_draws(n, seed):
    out = np.empty(n, np.float32)
    synth().pz_synth_draws(_np_ptr(out), n, seed)
    return out


def synth_draft_ids(draft, tau, seed):
    rows, V = draft.shape
    out = np.empty(rows, np.int32)
    synth().pz_synth_draft_ids(_np_ptr(out), _np_ptr(np.ascontiguousarray(draft)), rows, V,
                               V, tau, seed)
    return out


PZ_NOALLOC_MAX_BATCH, PZ_NOALLOC_MAX_VOCAB, PZ_NOALLOC_MAX_HIST = 64, 262144, 2048
PZ_ID_FAILED = -2  # a row whose wait between workgroups gave up


def sample_noalloc(d_logits, B, V, ld, params, d_u, d_ids, d_p=None, d_hist=None, H=0,
                   device=0, stream=None, temp_mode=PZ_TEMP_MUL_RECIP):
    """pz_sample_batch_noalloc: enqueues the batch on `stream` (a hipStream_t
    address, None for the null stream) without a sampler object; uniforms,
    ids and p are device buffers.  Returns the status code (PZ_OK or PZ_E*)."""
    lib = load()
    parr, n = _params_array(params, B)
    return lib.pz_sample_batch_noalloc(device, stream, temp_mode, _ptr(d_logits), B, V, ld,
                                       parr, n, _ptr(d_hist), H, _ptr(d_u), _ptr(d_ids),
                                       _ptr(d_p))
