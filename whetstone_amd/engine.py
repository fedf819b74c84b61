"""Python handle on the C++ decode engine (include/whetstone_engine.h).

The engine restates the reference's Engine (crates/whetstone-core/src/engine.rs)
over the C ABI; this module only binds it. There is no Python or CPU fallback:
a missing library raises.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import ffi

STEP_REFERENCE = 0
STEP_FUSED = 1
STAGES = ["embed", "qkv", "attn", "o", "gate_up", "down", "head", "rescore", "sample"]


class Config(C.Structure):
    """wse_config_t; field order matches oracle.Config."""
    _fields_ = [
        ("n_layers", C.c_int32), ("hidden", C.c_int32), ("n_q", C.c_int32),
        ("n_kv", C.c_int32), ("head_dim", C.c_int32), ("inter", C.c_int32),
        ("vocab", C.c_int32), ("tied", C.c_int32), ("qkv_bias", C.c_int32),
        ("qk_norm", C.c_int32), ("rescore_k", C.c_int32), ("eps", C.c_float),
        ("rope_theta", C.c_double), ("rope_llama3", C.c_int32), ("rope_orig_max", C.c_int32),
        ("rope_factor", C.c_double), ("rope_low_freq", C.c_double),
        ("rope_high_freq", C.c_double),
    ]


# Shapes of BASELINE.json's configurations (config.rs conventions).
QWEN05B = dict(n_layers=24, hidden=896, n_q=14, n_kv=2, head_dim=64, inter=4864,
               vocab=151936, tied=1, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6,
               rope_theta=1e6)
QWEN7B = dict(n_layers=28, hidden=3584, n_q=28, n_kv=4, head_dim=128, inter=18944,
              vocab=152064, tied=0, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6,
              rope_theta=1e6)

P = C.c_void_p
PP = C.POINTER(C.c_void_p)
I32 = C.c_int32
_SIG = {
    "wse_last_error": (C.c_char_p, []),
    "wse_model_synthetic": (I32, [C.POINTER(Config), C.c_uint64, PP]),
    "wse_model_free": (None, [P]),
    "wse_model_tensor": (I32, [P, C.c_char_p, PP, PP, PP, C.POINTER(C.c_int64),
                               C.POINTER(C.c_int64)]),
    "wse_model_weight_bytes": (C.c_uint64, [P]),
    "wse_model_config": (I32, [P, C.POINTER(Config)]),
    "wse_model_vector": (I32, [P, C.c_char_p, PP, C.POINTER(C.c_int64)]),
    "wse_fnv1a": (C.c_uint64, [P, C.c_size_t]),
    "wse_wstone_check": (I32, [C.c_char_p, I32, C.POINTER(I32)]),
    "wse_wstone_config": (I32, [C.c_char_p, C.POINTER(Config)]),
    "wse_config_from_json": (I32, [C.c_char_p, C.POINTER(Config)]),
    "wse_model_load_wstone": (I32, [C.c_char_p, I32, PP]),
    "wse_engine_create": (I32, [P, I32, I32, PP]),
    "wse_engine_free": (None, [P]),
    "wse_engine_reset": (I32, [P]),
    "wse_engine_pos": (I32, [P]),
    "wse_engine_set_pos": (I32, [P, I32]),
    "wse_engine_fill_kv": (I32, [P, C.c_uint64, I32]),
    "wse_engine_forward": (I32, [P, I32]),
    "wse_engine_step": (I32, [P]),
    "wse_engine_capture_graph": (I32, [P]),
    "wse_engine_prefill": (I32, [P, P, I32, I32]),
    "wse_engine_generate": (I32, [P, P, I32, I32, I32, P, P]),
    "wse_engine_token": (I32, [P, C.POINTER(I32)]),
    "wse_engine_set_token": (I32, [P, I32]),
    "wse_engine_logits": (I32, [P, P]),
    "wse_engine_profile_step": (I32, [P, C.POINTER(C.c_double), C.POINTER(I32)]),
    "wse_engine_step_bytes": (C.c_uint64, [P]),
    "wse_engine_time_stage": (I32, [P, I32, I32, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    "wse_engine_max_seq": (I32, [P, C.POINTER(I32)]),
    "wse_engine_chunk_width": (I32, [P, C.POINTER(I32)]),
    "wse_engine_forward_chunk": (I32, [P, P, I32, I32]),
    "wse_engine_chunk_picks": (I32, [P, I32, P]),
    "wse_engine_rewind": (I32, [P, I32]),
    "wse_sample_with": (I32, [P, I32, P, C.c_uint64, P, I32]),
    "wse_splitmix64": (C.c_uint64, [C.c_uint64]),
    "wse_engine_sample": (I32, [P, P, C.c_uint64, C.POINTER(I32)]),
    "wse_engine_generate_sampled": (I32, [P, P, I32, I32, I32, P, P, C.POINTER(I32)]),
    "wse_engine_recent": (I32, [P, P, I32]),
    "wse_engine_unnote": (None, [P, I32]),
    "wse_engine_cross_entropy": (I32, [P, P, C.c_int64, I32, I32, C.POINTER(C.c_double),
                                       C.POINTER(C.c_int64)]),
    "wse_spec_propose": (I32, [P, I32, I32, I32, I32, P]),
    "wse_speculate_generate": (I32, [P, P, I32, I32, P, P, C.POINTER(I32), P]),
}


class SpecConfig(C.Structure):
    """wse_spec_config_t (speculate.rs SpecConfig); defaults of its Default."""
    _fields_ = [("draft", C.c_int32), ("ngram_max", C.c_int32), ("ngram_min", C.c_int32)]

    def __init__(self, draft: int = 4, ngram_max: int = 3, ngram_min: int = 2):
        super().__init__(draft, ngram_max, ngram_min)


class SamplingConfig(C.Structure):
    """SamplingConfig (engine.rs:104-137); the defaults are the reference's."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", I32),
                ("min_p", C.c_float), ("repeat_penalty", C.c_float), ("repeat_last_n", I32),
                ("seed", C.c_uint64)]

    def __init__(self, temperature=0.7, top_p=0.8, top_k=20, min_p=0.0, repeat_penalty=1.05,
                 repeat_last_n=64, seed=0):
        super().__init__(temperature, top_p, top_k, min_p, repeat_penalty, repeat_last_n, seed)


def sample_with(logits, cfg: "SamplingConfig", step: int, recent=()):
    """sample_with on a host copy: (token, the penalised logits)."""
    v = np.array(logits, np.float32, copy=True)
    r = np.ascontiguousarray(list(recent), np.int32)
    t = lib().wse_sample_with(v.ctypes.data, v.size, C.byref(cfg), step,
                              r.ctypes.data if r.size else None, r.size)
    return int(t), v


def splitmix64(z: int) -> int:
    return int(lib().wse_splitmix64(z))


class SpecStats(C.Structure):
    """wse_spec_stats_t (speculate.rs SpecStats)."""
    _fields_ = [("rounds", C.c_int64), ("empty_rounds", C.c_int64), ("proposed", C.c_int64),
                ("accepted", C.c_int64)]

    def acceptance(self) -> float:
        return self.accepted / self.proposed if self.proposed else 0.0

    def tokens_per_round(self) -> float:
        return (self.rounds + self.accepted) / self.rounds if self.rounds else 0.0


def spec_propose(history, ngram_max: int = 3, ngram_min: int = 2, want: int = 3) -> list[int]:
    """speculate.rs propose: the n-gram draft (host code in the engine library)."""
    h = np.ascontiguousarray(history, np.int32)
    out = np.zeros(max(want, 1), np.int32)
    n = lib().wse_spec_propose(h.ctypes.data, h.size, ngram_max, ngram_min, want, out.ctypes.data)
    return [int(v) for v in out[:n]]
_lib = None


def lib():
    global _lib
    if _lib is None:
        ffi.lib()  # the kernel library first (the engine links against it)
        if not ffi.ENGINE_LIB.exists():
            raise FileNotFoundError(f"{ffi.ENGINE_LIB} is missing; run python -m whetstone_amd.build")
        L = C.CDLL(str(ffi.ENGINE_LIB))
        for name, (res, args) in _SIG.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(st: int) -> None:
    if st != ffi.WST_OK:
        msg = lib().wse_last_error().decode(errors="replace")
        kmsg = ffi.lib().wst_last_error().decode(errors="replace")
        raise ffi.WstError(st, f"{msg} | {kmsg}")


def _config_dict(c: Config) -> dict:
    return {name: getattr(c, name) for name, _ in Config._fields_}


def config_from_json(text: str) -> dict:
    """A config.json parsed and validated as the loader does (config.rs)."""
    c = Config()
    _check(lib().wse_config_from_json(text.encode(), C.byref(c)))
    return _config_dict(c)


def wstone_check(path, verify: bool = False) -> int:
    """Validates a .wstone file's header (and, with verify, every payload
    hash); returns the tensor count. Raises WstError with the reason."""
    n = C.c_int32()
    _check(lib().wse_wstone_check(str(path).encode(), int(verify), C.byref(n)))
    return n.value


def wstone_config(path) -> dict:
    c = Config()
    _check(lib().wse_wstone_config(str(path).encode(), C.byref(c)))
    return _config_dict(c)


class Model:
    """Device-resident weights: seeded synthetic ones generated and packed in
    HBM, or a .wstone file loaded with Model.load."""

    def __init__(self, cfg: dict | None, seed: int = 0, _handle=None):
        if _handle is not None:
            self.h = _handle
            c = Config()
            _check(lib().wse_model_config(self.h, C.byref(c)))
            self.cfg = _config_dict(c)
            self._c = c
            return
        self.cfg = dict(cfg)
        self._c = Config(**self.cfg)
        h = C.c_void_p()
        _check(lib().wse_model_synthetic(C.byref(self._c), seed, C.byref(h)))
        self.h = h

    @classmethod
    def load(cls, path, rescore_k: int = -1) -> "Model":
        """Loads a .wstone file (model.rs:454-638); rescore_k < 0 enables the
        top-64 rescore when the file carries the head's f16 copy."""
        h = C.c_void_p()
        _check(lib().wse_model_load_wstone(str(path).encode(), rescore_k, C.byref(h)))
        return cls(None, _handle=h)

    def vector_host(self, name: str) -> np.ndarray:
        """An f16 tensor of the model (norm gains, biases, the head copy) as
        f16 bit patterns on the host."""
        p, n = C.c_void_p(), C.c_int64()
        _check(lib().wse_model_vector(self.h, name.encode(), C.byref(p), C.byref(n)))
        out = np.empty(n.value, np.uint16)
        ffi.check(ffi.lib().wst_memcpy_d2h(out.ctypes.data, p.value, out.nbytes))
        return out

    def tensor(self, name: str):
        qw, si, sb = C.c_void_p(), C.c_void_p(), C.c_void_p()
        i, o = C.c_int64(), C.c_int64()
        _check(lib().wse_model_tensor(self.h, name.encode(), C.byref(qw), C.byref(si),
                                      C.byref(sb), C.byref(i), C.byref(o)))
        return qw.value, si.value, sb.value, i.value, o.value

    def tensor_host(self, name: str, rows=None):
        """Copies (a row range of) a packed matrix to the host."""
        qw, si, sb, i, o = self.tensor(name)
        r0, r1 = (0, o) if rows is None else rows
        n = r1 - r0
        q = np.empty(n * i // 8, np.uint32)
        s = np.empty(n * i // 32, np.uint8)
        b = np.empty(n, np.uint32)
        ffi.check(ffi.lib().wst_memcpy_d2h(q.ctypes.data, qw + r0 * i // 2, q.nbytes))
        ffi.check(ffi.lib().wst_memcpy_d2h(s.ctypes.data, si + r0 * i // 32, s.nbytes))
        ffi.check(ffi.lib().wst_memcpy_d2h(b.ctypes.data, sb + r0 * 4, b.nbytes))
        return q, s, b, i, n

    def weight_bytes(self) -> int:
        return int(lib().wse_model_weight_bytes(self.h))

    def close(self):
        if self.h is not None and self.h.value:
            lib().wse_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Engine:
    def __init__(self, model: Model, max_seq: int, mode: int = STEP_FUSED):
        self.model = model
        h = C.c_void_p()
        _check(lib().wse_engine_create(model.h, max_seq, mode, C.byref(h)))
        self.h = h
        self.max_seq = max_seq
        self.vocab = model.cfg["vocab"]

    @property
    def pos(self) -> int:
        return int(lib().wse_engine_pos(self.h))

    def set_pos(self, p: int):
        _check(lib().wse_engine_set_pos(self.h, p))

    def reset(self):
        _check(lib().wse_engine_reset(self.h))

    def fill_kv(self, seed: int, n: int):
        _check(lib().wse_engine_fill_kv(self.h, seed, n))

    def forward(self, token: int):
        _check(lib().wse_engine_forward(self.h, token))

    def step(self):
        _check(lib().wse_engine_step(self.h))

    def capture_graph(self):
        _check(lib().wse_engine_capture_graph(self.h))

    def prefill(self, ids, chunked: bool = True):
        a = np.ascontiguousarray(ids, np.int32)
        _check(lib().wse_engine_prefill(self.h, a.ctypes.data, a.size, int(chunked)))

    def generate(self, prompt, n_new: int, chunked: bool = True) -> np.ndarray:
        a = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        n = C.c_int32()
        _check(lib().wse_engine_generate(self.h, a.ctypes.data, a.size, n_new, int(chunked),
                                         out.ctypes.data, C.byref(n)))
        return out[:n.value]

    def chunk_width(self) -> int:
        w = C.c_int32()
        _check(lib().wse_engine_chunk_width(self.h, C.byref(w)))
        return w.value

    def forward_chunk(self, ids, want_logits: bool = True):
        a = np.ascontiguousarray(ids, np.int32)
        _check(lib().wse_engine_forward_chunk(self.h, a.ctypes.data, a.size, int(want_logits)))

    def chunk_picks(self, n: int) -> np.ndarray:
        out = np.zeros(max(n, 1), np.int32)
        _check(lib().wse_engine_chunk_picks(self.h, n, out.ctypes.data))
        return out[:n]

    def rewind(self, pos: int):
        _check(lib().wse_engine_rewind(self.h, pos))

    def speculate(self, prompt, max_new: int, cfg: SpecConfig | None = None):
        """speculate::generate: (tokens, SpecStats)."""
        a = np.ascontiguousarray(prompt, np.int32)
        cfg = SpecConfig() if cfg is None else cfg
        out = np.zeros(max(max_new, 1), np.int32)
        n, st = C.c_int32(), SpecStats()
        _check(lib().wse_speculate_generate(self.h, a.ctypes.data, a.size, max_new, C.byref(cfg),
                                            out.ctypes.data, C.byref(n), C.byref(st)))
        return out[:n.value], st

    def cross_entropy(self, tokens, window: int, max_windows: int = 1 << 30):
        """Engine::cross_entropy: (summed NLL in nats, predicted positions)."""
        a = np.ascontiguousarray(tokens, np.int32)
        nll, n = C.c_double(), C.c_int64()
        _check(lib().wse_engine_cross_entropy(self.h, a.ctypes.data, a.size, window, max_windows,
                                              C.byref(nll), C.byref(n)))
        return nll.value, n.value

    def sample(self, cfg: "SamplingConfig | None", step: int) -> int:
        """Engine::sample: None is Sampler::Greedy."""
        t = C.c_int32()
        _check(lib().wse_engine_sample(self.h, C.byref(cfg) if cfg is not None else None, step,
                                       C.byref(t)))
        return t.value

    def generate_sampled(self, prompt, n_new: int, cfg: "SamplingConfig | None",
                         chunked: bool = True) -> np.ndarray:
        a = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        n = C.c_int32()
        _check(lib().wse_engine_generate_sampled(self.h, a.ctypes.data, a.size, n_new,
                                                 int(chunked),
                                                 C.byref(cfg) if cfg is not None else None,
                                                 out.ctypes.data, C.byref(n)))
        return out[:n.value]

    def recent(self) -> list:
        n = lib().wse_engine_recent(self.h, None, 0)
        out = np.zeros(max(n, 1), np.int32)
        lib().wse_engine_recent(self.h, out.ctypes.data, n)
        return [int(v) for v in out[:n]]

    def set_token(self, token: int):
        _check(lib().wse_engine_set_token(self.h, token))

    def token(self) -> int:
        t = C.c_int32()
        _check(lib().wse_engine_token(self.h, C.byref(t)))
        return t.value

    def logits(self) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        _check(lib().wse_engine_logits(self.h, out.ctypes.data))
        return out

    def profile_step(self, acc=None, counts=None):
        acc = np.zeros(len(STAGES), np.float64) if acc is None else acc
        counts = np.zeros(len(STAGES), np.int32) if counts is None else counts
        _check(lib().wse_engine_profile_step(
            self.h, acc.ctypes.data_as(C.POINTER(C.c_double)),
            counts.ctypes.data_as(C.POINTER(C.c_int32))))
        return acc, counts

    def time_stage(self, stage: str, reps: int = 20):
        """(µs per launch, algorithmic bytes per launch) of one stage's kernel."""
        us, b = C.c_double(), C.c_uint64()
        _check(lib().wse_engine_time_stage(self.h, STAGES.index(stage), reps, C.byref(us),
                                           C.byref(b)))
        return us.value, int(b.value)

    def step_bytes(self) -> int:
        return int(lib().wse_engine_step_bytes(self.h))

    def close(self):
        if self.h is not None and self.h.value:
            lib().wse_engine_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
