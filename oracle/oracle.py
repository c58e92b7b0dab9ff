"""ctypes wrapper of the CPU oracle (liboracle.so built from g2_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by bench.py's CPU-baseline leg, as the test reference or as the timed CPU
baseline.
The shipped library (gpt2-opencl-1.1_amd/) never imports it.

Functions take and return numpy arrays; names follow the reference kernels
(math.cl) and host functions (main.c) they restate.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")


def build():
    subprocess.run(["make", "-B", "-C", _HERE], check=True, stdout=subprocess.DEVNULL)


if not os.path.exists(LIB_PATH):
    build()
_lib = C.CDLL(LIB_PATH)

_vp, _i, _f = C.c_void_p, C.c_int, C.c_float
for _n, _a, _r in [
    ("or_matmul", [_vp, _vp, _vp, _vp, _i, _i, _i], None),
    ("or_matvec", [_vp, _vp, _vp, _vp, _vp, _i, _i, _i], None),
    ("or_matvec4", [_vp, _vp, _vp, _vp, _vp, _i, _i, _i], None),
    ("or_matvec4_sk", [_vp, _vp, _vp, _i, _i, _i], None),
    ("or_reduce_partial", [_vp, _vp, _vp, _vp, _i, _i, _i], None),
    ("or_layernorm", [_vp, _vp, _vp, _vp, _i, _i], None),
    ("or_add_inplace", [_vp, _vp, _i], None),
    ("or_gelu", [_vp, _i], None),
    ("or_embed", [_vp, _vp, _vp, _i, _i, _i, _vp], None),
    ("or_split_kv", [_vp, _vp, _vp, _i, _i, _i, _i], None),
    ("or_attn_scores_1q", [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f], None),
    ("or_attn_softmax_1q", [_vp, _i, _i, _i, _i], None),
    ("or_attn_out_1q", [_vp, _vp, _vp, _i, _i, _i, _i, _i], None),
    ("or_model_create", [_i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp], _vp),
    ("or_model_destroy", [_vp], None),
    ("or_model_set_lm_head", [_vp, _vp], None),
    ("or_prefill", [_vp, _vp, _i], None),
    ("or_decode", [_vp, _i, _i], None),
    ("or_logits", [_vp], C.POINTER(C.c_float)),
    ("or_greedy", [_vp, _i, _vp, _i, _i, _f, _vp], _i),
    ("or_generate", [_vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp, _i], _i),
    ("or_teacher_forced", [_vp, _vp, _i, _vp, _i, _vp], None),
    ("or_set_kv", [_vp, _i, _vp, _vp], None),
    ("or_num_threads", [], _i),
]:
    fn = getattr(_lib, _n)
    fn.argtypes = _a
    fn.restype = _r


def num_threads():
    """OpenMP threads the oracle runs with (OMP_NUM_THREADS or all cores)."""
    return _lib.or_num_threads()


def _a32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _ptr(x):
    return None if x is None else x.ctypes.data


def matmul(A, B, bias, M, N, K):
    A, B = _a32(A), _a32(B)
    bias = None if bias is None else _a32(bias)
    Cm = np.empty((M, N), np.float32)
    _lib.or_matmul(_ptr(A), _ptr(B), _ptr(bias), _ptr(Cm), M, N, K)
    return Cm


def matvec(A, B, bias, residual, N, K, apply_gelu=0):
    """launch_matvec semantics: matvec4 when N%4==0, scalar matvec otherwise."""
    A, B = _a32(A), _a32(B)
    bias = None if bias is None else _a32(bias)
    residual = None if residual is None else _a32(residual)
    out = np.empty(N, np.float32)
    fn = _lib.or_matvec4 if N % 4 == 0 else _lib.or_matvec
    fn(_ptr(A), _ptr(B), _ptr(bias), _ptr(residual), _ptr(out), N, K, int(apply_gelu))
    return out


def matvec_scalar(A, B, bias, residual, N, K, apply_gelu=0):
    A, B = _a32(A), _a32(B)
    bias = None if bias is None else _a32(bias)
    residual = None if residual is None else _a32(residual)
    out = np.empty(N, np.float32)
    _lib.or_matvec(_ptr(A), _ptr(B), _ptr(bias), _ptr(residual), _ptr(out), N, K, int(apply_gelu))
    return out


def matvec4_sk(A, B, N, K, kslice):
    A, B = _a32(A), _a32(B)
    part = np.empty((kslice, N), np.float32)
    _lib.or_matvec4_sk(_ptr(A), _ptr(B), _ptr(part), N, K, kslice)
    return part


def reduce_partial(partial, bias, residual, N, kslice, apply_gelu=0):
    partial = _a32(partial)
    bias = None if bias is None else _a32(bias)
    residual = None if residual is None else _a32(residual)
    out = np.empty(N, np.float32)
    _lib.or_reduce_partial(_ptr(partial), _ptr(bias), _ptr(residual), _ptr(out), N, kslice, int(apply_gelu))
    return out


def layernorm(x, gamma, beta, n_embd, seq_len):
    x = _a32(x)
    out = np.empty_like(x)
    _lib.or_layernorm(_ptr(x), _ptr(out), _ptr(_a32(gamma)), _ptr(_a32(beta)), n_embd, seq_len)
    return out


def add_inplace(a, b):
    a = _a32(a).copy()
    _lib.or_add_inplace(_ptr(a), _ptr(_a32(b)), a.size)
    return a


def gelu(x):
    x = _a32(x).copy()
    _lib.or_gelu(_ptr(x), x.size)
    return x


def embed(wte, wpe, n_embd, seq_len, start_pos, ids):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((seq_len, n_embd), np.float32)
    _lib.or_embed(_ptr(_a32(wte)), _ptr(_a32(wpe)), _ptr(out), n_embd, seq_len, start_pos, _ptr(ids))
    return out


def split_kv(qkv, k_cache, v_cache, start_pos, T, D, max_seq):
    """Returns updated copies of the caches."""
    kc, vc = _a32(k_cache).copy(), _a32(v_cache).copy()
    _lib.or_split_kv(_ptr(_a32(qkv)), _ptr(kc), _ptr(vc), start_pos, T, D, max_seq)
    return kc, vc


def attn_scores_1q(qkv, k_cache, q_base, T_kv, D, DH, NH, max_seq, scale):
    scores = np.zeros((NH, max_seq), np.float32)
    _lib.or_attn_scores_1q(_ptr(_a32(qkv)), _ptr(_a32(k_cache)), _ptr(scores), q_base, T_kv, D, DH,
                           NH, max_seq, scale)
    return scores


def attn_softmax_1q(scores, T_kv, NH, row_stride=1024, lws=64):
    s = _a32(scores).copy()
    _lib.or_attn_softmax_1q(_ptr(s), T_kv, NH, row_stride, lws)
    return s


def attn_out_1q(scores, v_cache, T_kv, D, DH, out_base, out_len, row_stride=1024):
    out = np.zeros(out_len, np.float32)
    _lib.or_attn_out_1q(_ptr(_a32(scores)), _ptr(_a32(v_cache)), _ptr(out), T_kv, D, DH, out_base,
                        row_stride)
    return out


class Model:
    """Oracle GPT-2 over host weights in the Conv1D [in,out] layout (the dict
    of g2hip.synth_weights; an optional "lm_head" [V, E] entry replaces the
    tied head).  kslice pins the split-K slice count of the
    attn_proj / ffn2 matvecs (the reference tunes it at start-up)."""

    def __init__(self, cfg, weights, kslice=4):
        self.cfg = cfg
        self._keep = []

        def ptr(a):
            a = _a32(a)
            self._keep.append(a)
            return a.ctypes.data

        flat = (_vp * (12 * cfg.n_layer))()
        for l, lw in enumerate(weights["layers"]):
            for s, a in enumerate(lw):
                flat[12 * l + s] = ptr(a)
        self._flat = flat
        self.h = _lib.or_model_create(cfg.n_layer, cfg.n_embd, cfg.n_head, cfg.vocab_size,
                                      cfg.ffn_dim, kslice, ptr(weights["wte"]), ptr(weights["wpe"]),
                                      ptr(weights["lnf_w"]), ptr(weights["lnf_b"]), flat)
        if weights.get("lm_head") is not None:  # separate [V, E] head instead of the tied wte
            _lib.or_model_set_lm_head(self.h, ptr(weights["lm_head"]))
        self.padded_vocab = (cfg.vocab_size + 3) & ~3

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.or_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        _lib.or_prefill(self.h, _ptr(ids), len(ids))

    def decode(self, token, pos):
        _lib.or_decode(self.h, int(token), int(pos))

    def set_kv(self, layer, k_cache, v_cache):
        k, v = _a32(k_cache), _a32(v_cache)
        assert k.size == v.size == self.cfg.n_embd * 1024
        _lib.or_set_kv(self.h, layer, _ptr(k), _ptr(v))

    def logits(self):
        p = _lib.or_logits(self.h)
        return np.ctypeslib.as_array(p, shape=(self.padded_vocab,))[: self.cfg.vocab_size].copy()

    def greedy(self, ctx, forbid_eos=False, rep_penalty=1.0):
        ctx = np.ascontiguousarray(ctx, dtype=np.int32)
        work = np.empty(self.padded_vocab, np.float32)
        lg = self.logits()
        return _lib.or_greedy(_ptr(lg), self.cfg.vocab_size, _ptr(ctx), len(ctx), int(forbid_eos),
                              rep_penalty, _ptr(work))

    def generate(self, prompt, max_new, min_new=None, rep_penalty=1.0, logit_steps=0):
        """Greedy generation loop of main.c:2106-2150.  Returns (ids,
        top2[n,2] = (chosen logit, runner-up) after masking, logits of the
        first `logit_steps` tokens [logit_steps, V])."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        min_new = max_new if min_new is None else min_new
        out = np.empty(1024, np.int32)
        top2 = np.empty((1024, 2), np.float32)
        lg = np.empty((max(logit_steps, 1), self.padded_vocab), np.float32)
        n = _lib.or_generate(self.h, _ptr(prompt), len(prompt), max_new, min_new, rep_penalty,
                             _ptr(out), _ptr(top2), _ptr(lg), logit_steps)
        return out[:n].copy(), top2[:n].copy(), lg[:logit_steps, : self.cfg.vocab_size].copy()

    def teacher_forced(self, prompt, forced):
        """Logits after prefill and after each forced decode token
        [len(forced)+1, V]."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        forced = np.ascontiguousarray(forced, dtype=np.int32)
        out = np.empty((len(forced) + 1, self.padded_vocab), np.float32)
        _lib.or_teacher_forced(self.h, _ptr(prompt), len(prompt), _ptr(forced), len(forced), _ptr(out))
        return out[:, : self.cfg.vocab_size].copy()
