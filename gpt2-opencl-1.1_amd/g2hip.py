"""ctypes binding of libg2hip.so, the C ABI declared in include/g2hip.h.

Mirrors the reference's operator surface (main.c launch_* helpers, math.cl
kernels) with the same names and argument meaning, plus the model entry
points (prefill/decode/greedy/generate).  Device buffers are `DevBuf`
objects (a device pointer and a byte size).  Every failing call raises
`G2Error` carrying the library's error code and message.

The library must have been built in this directory (`make -B` here, or
`__graft_entry__.build()`); importing this module without it raises
ImportError -- there is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libg2hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "g2hip.h")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built; run make in {_HERE}")
_lib = C.CDLL(LIB_PATH)

G2_OK, G2_E_ARG, G2_E_STATE, G2_E_IO, G2_E_FORMAT, G2_E_LIMIT, G2_E_NOMEM, G2_E_HIP = 0, -1, -2, -3, -4, -5, -6, -7
F32, F16 = 0, 1
PATH_REFERENCE, PATH_FUSED = 0, 1
MAX_SEQ = 1024
EOS = 50256


class G2Error(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"g2 error {code}: {msg}")
        self.code = code


class Config(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("n_embd", C.c_int), ("n_head", C.c_int),
                ("n_ctx", C.c_int), ("vocab_size", C.c_int), ("ffn_dim", C.c_int)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


def make_config(n_layer, n_embd, n_head, vocab_size=50257, ffn_dim=None, n_ctx=1024):
    return Config(n_layer, n_embd, n_head, n_ctx, vocab_size, ffn_dim or 4 * n_embd)


PRESETS = {
    "small": (12, 768, 12), "medium": (24, 1024, 16),
    "large": (36, 1280, 20), "xl": (48, 1600, 25),
}


def preset(name):
    L, E, H = PRESETS[name]
    return make_config(L, E, H)


_vp = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t


def _sig(name, res, *args):
    fn = getattr(_lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


_sig("g2_last_error", C.c_char_p)
for _n, _a in {
    "g2_init": [_i], "g2_shutdown": [], "g2_device_name": [C.c_char_p, _i, C.POINTER(_i)],
    "g2_alloc": [C.POINTER(_vp), _sz], "g2_free": [_vp], "g2_upload": [_vp, _vp, _sz],
    "g2_upload_rect": [_vp, _sz, _vp, _sz, _sz, _sz], "g2_copy": [_vp, _vp, _sz],
    "g2_download": [_vp, _vp, _sz], "g2_memset": [_vp, _i, _sz], "g2_sync": [],
    "g2_matmul": [_vp, _vp, _vp, _vp, _i, _i, _i], "g2_matmul_f16": [_vp, _vp, _vp, _vp, _i, _i, _i],
    "g2_matvec": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i],
    "g2_matvec_f16": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i],
    "g2_matvec_sk": [_vp, _vp, _vp, _i, _i, _i], "g2_matvec_sk_f16": [_vp, _vp, _vp, _i, _i, _i],
    "g2_reduce_partial": [_vp, _vp, _vp, _vp, _i, _i, _i],
    "g2_layernorm": [_vp, _vp, _vp, _vp, _i, _i], "g2_add": [_vp, _vp, _i], "g2_gelu": [_vp, _i],
    "g2_embed": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "g2_split_kv": [_vp, _vp, _vp, _i, _i, _i, _i],
    "g2_attn_scores_1q": [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f],
    "g2_attn_softmax_1q": [_vp, _i, _i], "g2_attn_out_1q": [_vp, _vp, _vp, _i, _i, _i, _i],
    "g2_attn_1q": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f],
    "g2_attn_1q_noalloc": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f],
    "g2_matvec_rows": [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i],
    "g2_model_uses_graph": [_vp], "g2_read_kv": [_vp, _i, _vp, _vp],
    "g2_config_load": [C.c_char_p, C.POINTER(Config)], "g2_config_parse": [C.c_char_p, C.POINTER(Config)],
    "g2_model_load": [C.c_char_p, _i, _i, C.POINTER(_vp)],
    "g2_model_synth": [C.POINTER(Config), C.c_uint64, _i, _i, C.POINTER(_vp)],
    "g2_model_from_host": [C.POINTER(Config), _vp, _vp, _vp, _vp, C.POINTER(_vp), _i, _i, C.POINTER(_vp)],
    "g2_model_free": [_vp], "g2_model_config": [_vp, C.POINTER(Config)],
    "g2_model_set_kslice": [_vp, _i], "g2_model_set_step": [_vp, _i], "g2_model_uses_step": [_vp],
    "g2_prefill": [_vp, _vp, _i], "g2_decode": [_vp, _i, _i], "g2_read_logits": [_vp, _vp, _i],
    "g2_sample_greedy": [_vp, _vp, _i, _i, _f],
    "g2_generate": [_vp, _vp, _i, _i, _i, _vp, C.POINTER(C.c_double)],
    "g2_decode_run": [_vp, _i, _i, _i, _i, _vp, C.POINTER(C.c_double)],
}.items():
    _sig(_n, _i, *_a)
_sig("g2_synth_normal", None, _vp, _sz, C.c_uint64, C.c_uint32, _f)
_sig("g2_synth_tensor_id", C.c_uint32, _i, _i)
_sig("g2_convert_f16", None, _vp, _vp, _sz)
_sig("g2_model_weight_bytes", _sz, _vp)
_sig("g2_model_step_kernel", C.c_char_p, _vp)
_sig("g2_stream", _vp)


def last_error():
    return _lib.g2_last_error().decode(errors="replace")


def check(rc):
    if rc < 0:
        raise G2Error(rc, last_error())
    return rc


def exported_symbols():
    """Names of every function prototype declared in include/g2hip.h."""
    import re
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g2_[a-z0-9_]+)\s*\(", text)))


# ---------------------------------------------------------------- runtime

def init(device=0):
    check(_lib.g2_init(device))


def shutdown():
    check(_lib.g2_shutdown())


def device_name():
    buf = C.create_string_buffer(256)
    cus = C.c_int(0)
    check(_lib.g2_device_name(buf, 256, C.byref(cus)))
    return buf.value.decode(), cus.value


def sync():
    check(_lib.g2_sync())


class DevBuf:
    """A device allocation (freed explicitly or when garbage-collected)."""

    def __init__(self, nbytes):
        p = _vp()
        check(_lib.g2_alloc(C.byref(p), nbytes))
        self.ptr = p.value
        self.nbytes = nbytes

    @property
    def value(self):
        return self.ptr

    def free(self):
        if self.ptr:
            _lib.g2_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def offset(self, nbytes):
        """Raw device pointer nbytes into the buffer (no ownership)."""
        return self.ptr + nbytes

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(_lib.g2_upload(self.ptr, arr.ctypes.data, arr.nbytes))
        return self

    def download(self, dtype=np.float32, count=None):
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        check(_lib.g2_download(out.ctypes.data, self.ptr, out.nbytes))
        return out


def to_device(arr):
    arr = np.ascontiguousarray(arr)
    return DevBuf(max(arr.nbytes, 4)).upload(arr)


def _p(x):
    if x is None:
        return None
    if isinstance(x, DevBuf):
        return x.ptr
    return int(x)


# ---------------------------------------------------------------- operators

def matmul(A, B, bias, Cb, M, N, K, f16=False):
    fn = _lib.g2_matmul_f16 if f16 else _lib.g2_matmul
    check(fn(_p(A), _p(B), _p(bias), _p(Cb), M, N, K))


def matvec(A, B, bias, residual, Cb, N, K, apply_gelu=0, f16=False):
    fn = _lib.g2_matvec_f16 if f16 else _lib.g2_matvec
    check(fn(_p(A), _p(B), _p(bias), _p(residual), _p(Cb), N, K, int(apply_gelu)))


def matvec_sk(A, B, partial, N, K, kslice, f16=False):
    fn = _lib.g2_matvec_sk_f16 if f16 else _lib.g2_matvec_sk
    check(fn(_p(A), _p(B), _p(partial), N, K, kslice))


def attn_1q_noalloc(qkv, k_cache, v_cache, out, q_base, T_kv, D, NH, max_seq, out_base, scale):
    """attn_1q with its chunk partials in the library's static device scratch."""
    check(_lib.g2_attn_1q_noalloc(_p(qkv), _p(k_cache), _p(v_cache), _p(out), q_base, T_kv, D, NH,
                                  max_seq, out_base, scale))


def matvec_rows(x, W, w_dtype, bias, residual, y, N, K, apply_gelu=0):
    """Packed (output-major W[N,K]) matvec of the fused model."""
    check(_lib.g2_matvec_rows(_p(x), _p(W), w_dtype, _p(bias), _p(residual), _p(y), N, K, int(apply_gelu)))


def reduce_partial(partial, bias, residual, Cb, N, kslice, apply_gelu=0):
    check(_lib.g2_reduce_partial(_p(partial), _p(bias), _p(residual), _p(Cb), N, kslice, int(apply_gelu)))


def layernorm(x, out, gamma, beta, n_embd, seq_len):
    check(_lib.g2_layernorm(_p(x), _p(out), _p(gamma), _p(beta), n_embd, seq_len))


def add(a, b, n):
    check(_lib.g2_add(_p(a), _p(b), n))


def gelu(x, n):
    check(_lib.g2_gelu(_p(x), n))


def embed(wte, wpe, out, n_embd, seq_len, start_pos, ids):
    check(_lib.g2_embed(_p(wte), _p(wpe), _p(out), n_embd, seq_len, start_pos, _p(ids)))


def split_kv(qkv, k_cache, v_cache, start_pos, T, D, max_seq):
    check(_lib.g2_split_kv(_p(qkv), _p(k_cache), _p(v_cache), start_pos, T, D, max_seq))


def attn_scores_1q(qkv, k_cache, scores, q_base, T_kv, D, DH, NH, max_seq, scale):
    check(_lib.g2_attn_scores_1q(_p(qkv), _p(k_cache), _p(scores), q_base, T_kv, D, DH, NH, max_seq, scale))


def attn_softmax_1q(scores, T_kv, NH):
    check(_lib.g2_attn_softmax_1q(_p(scores), T_kv, NH))


def attn_out_1q(scores, v_cache, out, T_kv, D, DH, out_base):
    check(_lib.g2_attn_out_1q(_p(scores), _p(v_cache), _p(out), T_kv, D, DH, out_base))


def attn_1q(qkv, k_cache, v_cache, out, q_base, T_kv, D, NH, max_seq, out_base, scale):
    check(_lib.g2_attn_1q(_p(qkv), _p(k_cache), _p(v_cache), _p(out), q_base, T_kv, D, NH,
                          max_seq, out_base, scale))


# ---------------------------------------------------------------- host-only

def config_parse(json_text):
    cfg = Config()
    check(_lib.g2_config_parse(json_text.encode(), C.byref(cfg)))
    return cfg


def config_load(directory):
    cfg = Config()
    check(_lib.g2_config_load(directory.encode(), C.byref(cfg)))
    return cfg


def synth_normal(n, seed, tensor_id, std=0.02):
    out = np.empty(n, dtype=np.float32)
    _lib.g2_synth_normal(out.ctypes.data, n, seed, tensor_id, std)
    return out


def synth_tensor_id(layer, which):
    return _lib.g2_synth_tensor_id(layer, which)


def convert_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    _lib.g2_convert_f16(out.ctypes.data, x.ctypes.data, x.size)
    return out


LAYER_SLOTS = ("ln1_w", "ln1_b", "qkv_w", "qkv_b", "proj_w", "proj_b", "ln2_w", "ln2_b", "fc_w", "fc_b",
               "fc2_w", "fc2_b")

# Scales of the affine parameters synth_weights(affine=True) draws: biases
# N(0, AFFINE_BIAS_STD), LayerNorm gamma 1 + N(0, AFFINE_LN_STD), beta N(0, AFFINE_LN_STD).
AFFINE_BIAS_STD = 0.02
AFFINE_LN_STD = 0.1


def synth_weights(cfg, seed, f16_round=False, affine=False):
    """Host copy of the synthetic random-init weights g2_model_synth builds:
    dict with wte [V,E], wpe [1024,E], lnf_w, lnf_b and `layers`, a list of
    12-tuples in LAYER_SLOTS order (ln1_w, ln1_b, qkv_w, qkv_b, proj_w,
    proj_b, ln2_w, ln2_b, fc_w, fc_b, fc2_w, fc2_b) with matrices in the
    Conv1D [in,out] layout.  With f16_round the matrices and embeddings are
    rounded to fp16 values (kept as float32), i.e. what the fp16 weight
    format stores.  With affine, every bias vector and LayerNorm gamma/beta
    (ln_1, ln_2, ln_f) is drawn at random instead of 0 / 1 / 0 (biases
    N(0, 0.02), gamma 1 + N(0, 0.1), beta N(0, 0.1), from a numpy generator
    seeded with `seed`), so each of them has a distinct, visible effect."""
    E, F, V = cfg.n_embd, cfg.ffn_dim, cfg.vocab_size

    def rnd(a):
        return a.astype(np.float16).astype(np.float32) if f16_round else a

    rng = np.random.default_rng(seed ^ 0x5A17) if affine else None

    def bias(n):
        if not affine:
            return np.zeros(n, np.float32)
        return (rng.standard_normal(n) * AFFINE_BIAS_STD).astype(np.float32)

    def gamma():
        if not affine:
            return np.ones(E, np.float32)
        return (1.0 + rng.standard_normal(E) * AFFINE_LN_STD).astype(np.float32)

    def beta():
        if not affine:
            return np.zeros(E, np.float32)
        return (rng.standard_normal(E) * AFFINE_LN_STD).astype(np.float32)

    wte = rnd(synth_normal(V * E, seed, synth_tensor_id(-1, 1)).reshape(V, E))
    wpe = rnd(synth_normal(MAX_SEQ * E, seed, synth_tensor_id(-1, 2)).reshape(MAX_SEQ, E))
    layers = []
    for l in range(cfg.n_layer):
        mats = []
        for w, (i, o) in enumerate([(E, 3 * E), (E, E), (E, F), (F, E)]):
            mats.append(rnd(synth_normal(i * o, seed, synth_tensor_id(l, w)).reshape(i, o)))
        layers.append((gamma(), beta(), mats[0], bias(3 * E), mats[1], bias(E),
                       gamma(), beta(), mats[2], bias(F), mats[3], bias(E)))
    return {"wte": wte, "wpe": wpe, "lnf_w": gamma(), "lnf_b": beta(), "layers": layers}


def swap_slots(weights, a, b, layer=None):
    """Copy of a synth_weights dict with layer slots a and b (LAYER_SLOTS
    names) exchanged in one layer (all layers if layer is None): a planted
    wiring mistake for checking that a parity test notices it."""
    ia, ib = LAYER_SLOTS.index(a), LAYER_SLOTS.index(b)
    out = dict(weights)
    layers = []
    for l, lw in enumerate(weights["layers"]):
        lw = list(lw)
        if layer is None or l == layer:
            lw[ia], lw[ib] = lw[ib], lw[ia]
        layers.append(tuple(lw))
    out["layers"] = layers
    return out


# ---------------------------------------------------------------- model

class Model:
    """A GPT-2 model resident on the GPU (g2_model handle)."""

    def __init__(self, handle, dtype=F32):
        self.h = handle
        self.dtype = dtype
        cfg = Config()
        check(_lib.g2_model_config(self.h, C.byref(cfg)))
        self.cfg = cfg

    @classmethod
    def synth(cls, cfg, seed, dtype=F32, path=PATH_FUSED):
        h = _vp()
        check(_lib.g2_model_synth(C.byref(cfg), seed, dtype, path, C.byref(h)))
        return cls(h.value, dtype)

    @classmethod
    def load(cls, directory, dtype=F32, path=PATH_FUSED):
        h = _vp()
        check(_lib.g2_model_load(directory.encode(), dtype, path, C.byref(h)))
        return cls(h.value, dtype)

    @classmethod
    def from_host(cls, cfg, weights, dtype=F32, path=PATH_FUSED):
        keep = []

        def ptr(a):
            a = np.ascontiguousarray(a, dtype=np.float32)
            keep.append(a)
            return a.ctypes.data

        flat = (_vp * (12 * cfg.n_layer))()
        for l, lw in enumerate(weights["layers"]):
            for s, a in enumerate(lw):
                flat[12 * l + s] = ptr(a)
        h = _vp()
        check(_lib.g2_model_from_host(C.byref(cfg), ptr(weights["wte"]), ptr(weights["wpe"]),
                                      ptr(weights["lnf_w"]), ptr(weights["lnf_b"]), flat,
                                      dtype, path, C.byref(h)))
        return cls(h.value, dtype)

    def free(self):
        if self.h:
            _lib.g2_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def set_kslice(self, ks):
        check(_lib.g2_model_set_kslice(self.h, ks))

    def weight_bytes(self):
        return _lib.g2_model_weight_bytes(self.h)

    def uses_graph(self):
        return _lib.g2_model_uses_graph(self.h)

    def set_step(self, on):
        """Decode with the persistent step kernel (True) or per-operator kernels."""
        check(_lib.g2_model_set_step(self.h, 1 if on else 0))

    def uses_step(self):
        return _lib.g2_model_uses_step(self.h) >= 1

    def step_kernel(self):
        """Name of the persistent step kernel this model launches, as the
        library reports it ("" when it decodes with per-operator kernels)."""
        return _lib.g2_model_step_kernel(self.h).decode()

    def step_kind(self):
        """1: persistent step kernel, 0: per-operator kernels."""
        return _lib.g2_model_uses_step(self.h)

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(_lib.g2_prefill(self.h, ids.ctypes.data, len(ids)))

    def decode(self, token, pos):
        check(_lib.g2_decode(self.h, int(token), int(pos)))

    def logits(self, n=None):
        n = self.cfg.vocab_size if n is None else n
        out = np.empty(n, dtype=np.float32)
        check(_lib.g2_read_logits(self.h, out.ctypes.data, n))
        return out

    def read_kv(self, layer):
        """(K [E,1024] transposed, V [1024,E]) of one layer."""
        E = self.cfg.n_embd
        k = np.empty((E, MAX_SEQ), np.float32)
        v = np.empty((MAX_SEQ, E), np.float32)
        check(_lib.g2_read_kv(self.h, layer, k.ctypes.data, v.ctypes.data))
        return k, v

    def sample_greedy(self, ctx, forbid_eos=False, rep_penalty=1.0):
        ctx = np.ascontiguousarray(ctx, dtype=np.int32)
        return check(_lib.g2_sample_greedy(self.h, ctx.ctypes.data, len(ctx), int(forbid_eos), rep_penalty))

    def generate(self, prompt, max_new, min_new=None):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        min_new = max_new if min_new is None else min_new
        out = np.empty(MAX_SEQ, dtype=np.int32)
        t = (C.c_double * 2)()
        n = check(_lib.g2_generate(self.h, prompt.ctypes.data, len(prompt), max_new, min_new,
                                   out.ctypes.data, t))
        return out[:n].copy(), (t[0], t[1])

    def decode_run(self, token, start_pos, n_steps, forbid_eos=True):
        out = np.empty(n_steps, dtype=np.int32)
        ms = C.c_double(0)
        check(_lib.g2_decode_run(self.h, int(token), int(start_pos), int(n_steps), int(forbid_eos),
                                 out.ctypes.data, C.byref(ms)))
        return out, ms.value


# ---------------------------------------------------------------- text

_sig("g2_tok_load", _i, C.c_char_p, C.POINTER(_vp))
_sig("g2_tok_free", None, _vp)
_sig("g2_tok_vocab_size", _i, _vp)
_sig("g2_tok_encode", _i, _vp, C.c_char_p, _vp, _i)
_sig("g2_tok_decode", _i, _vp, _vp, _i, _vp, _i)


class Tokenizer:
    """GPT-2 byte-level BPE over vocab.json + merges.txt in a directory,
    with the reference tokenizer's behaviour (tokenizer.c; gpt2_encode /
    gpt2_decode -> encode / decode).  Host-only: needs no device."""

    def __init__(self, directory):
        h = _vp()
        check(_lib.g2_tok_load(os.fsencode(str(directory)), C.byref(h)))
        self.h = h

    def free(self):
        if self.h:
            _lib.g2_tok_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def vocab_size(self):
        return _lib.g2_tok_vocab_size(self.h)

    def encode(self, text, max_ids=MAX_SEQ - 1):
        """ids of UTF-8 text (str or bytes without NUL), at most max_ids
        (main.c encodes prompts with MAX_SEQ_LEN - 1)."""
        raw = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        if b"\0" in raw:
            raise G2Error(G2_E_ARG, "text contains NUL")
        buf = np.empty(max(int(max_ids), 1), dtype=np.int32)
        n = _lib.g2_tok_encode(self.h, raw, buf.ctypes.data, int(max_ids))
        if n < 0:
            raise G2Error(G2_E_ARG, "g2_tok_encode: bad arguments")
        return buf[:n].copy()

    def decode(self, ids, max_bytes=None):
        """bytes of the ids (undecodable code points as '?'), truncated to
        max_bytes - 1 bytes (default: enough for every token)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        cap = int(max_bytes) if max_bytes is not None else 64 * max(len(ids), 1) + 1
        out = C.create_string_buffer(cap)
        n = _lib.g2_tok_decode(self.h, ids.ctypes.data, len(ids), out, cap)
        if n < 0:
            raise G2Error(G2_E_ARG, "g2_tok_decode: bad arguments")
        return out.raw[:n]

    def decode_text(self, ids):
        return self.decode(ids).decode("utf-8", errors="replace")
