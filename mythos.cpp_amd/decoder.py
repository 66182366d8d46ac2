"""ctypes binding of the decoder stack in libmythos_oil.so
(include/mythos_decoder.h).

`Decoder` plays the part of the reference's DenseModel + Generator
(src/model.cpp:45-75, src/generator.cpp:14-64) for the mixed-format stack:
weights are uploaded once into device memory owned by this object (torch
tensors: plumbing only), the library owns the KV cache and activations, and
`generate` feeds the prompt then greedy tokens one step at a time, each step
replayed from one captured HIP graph.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

import mythos_oil

_lib = mythos_oil.lib
VP, I64, I32, F32 = C.c_void_p, C.c_int64, C.c_int, C.c_float

EXPORTS = ("mth_decoder_create", "mth_decoder_destroy", "mth_decoder_set_layer", "mth_decoder_set_globals",
           "mth_decoder_start", "mth_decoder_step", "mth_decoder_buffers", "mth_decoder_read",
           "mth_decoder_steps_done", "mth_decoder_set_taps", "mth_decoder_tap_floats", "mth_decoder_read_kv",
           "mth_decoder_launches", "mth_decoder_prefill")

CONFIG_KEYS = ("vocab", "hidden", "layers", "heads", "kv_heads", "head_dim", "ffn", "max_seq", "cb_block",
               "max_batch")


class Config(C.Structure):
    _fields_ = [("struct_size", C.c_int64)] + [(k, C.c_int64) for k in CONFIG_KEYS] + \
               [("eps", C.c_float), ("theta", C.c_float), ("kv_dtype", C.c_int64)]


KV_DTYPES = {"f32": 0, "bf16": 1}


class Layer(C.Structure):
    _fields_ = [("attn_norm", VP), ("ffn_norm", VP), ("wq", VP), ("wk", VP), ("wv", VP), ("wo", VP),
                ("cbq", VP), ("cbk", VP), ("cbv", VP), ("cbo", VP), ("wgate", VP), ("wup", VP),
                ("cbgate", VP), ("cbup", VP), ("wdown", VP), ("down_scale", C.c_float)]


class Globals(C.Structure):
    _fields_ = [("emb", VP), ("final_norm", VP), ("lm_idx", VP), ("lm_cb", VP)]


_lib.mth_decoder_create.argtypes = [C.POINTER(Config), C.POINTER(VP)]
_lib.mth_decoder_create.restype = I32
_lib.mth_decoder_destroy.argtypes = [VP]
_lib.mth_decoder_destroy.restype = None
_lib.mth_decoder_set_layer.argtypes = [VP, I64, C.POINTER(Layer)]
_lib.mth_decoder_set_layer.restype = I32
_lib.mth_decoder_set_globals.argtypes = [VP, C.POINTER(Globals)]
_lib.mth_decoder_set_globals.restype = I32
_lib.mth_decoder_start.argtypes = [VP, VP, I64, I64, VP]
_lib.mth_decoder_start.restype = I32
_lib.mth_decoder_step.argtypes = [VP, I64, I32, VP]
_lib.mth_decoder_step.restype = I32
_lib.mth_decoder_buffers.argtypes = [VP, C.POINTER(VP), C.POINTER(VP), C.POINTER(I64)]
_lib.mth_decoder_buffers.restype = I32
_lib.mth_decoder_read.argtypes = [VP, VP, VP, VP]
_lib.mth_decoder_read.restype = I32
_lib.mth_decoder_steps_done.argtypes = [VP]
_lib.mth_decoder_steps_done.restype = I64
_lib.mth_decoder_prefill.argtypes = [VP, VP]
_lib.mth_decoder_launches.argtypes = [VP]
_lib.mth_decoder_launches.restype = I64
_lib.mth_decoder_set_taps.argtypes = [VP, VP]
_lib.mth_decoder_set_taps.restype = I32
_lib.mth_decoder_tap_floats.argtypes = [VP]
_lib.mth_decoder_tap_floats.restype = I64
_lib.mth_decoder_read_kv.argtypes = [VP, I64, VP, VP, VP]
_lib.mth_decoder_read_kv.restype = I32


def _check(rc):
    if rc != mythos_oil.MTH_OK:
        raise mythos_oil.MythosError(rc, mythos_oil.last_error())


class Decoder:
    def __init__(self, cfg: dict, max_batch: int = 1, device="cuda", kv_dtype: str = "f32"):
        self.cfg = dict(cfg, max_batch=max_batch)
        self.device = device
        self.kv_dtype = kv_dtype
        c = Config(C.sizeof(Config), *[int(self.cfg[k]) for k in CONFIG_KEYS], float(cfg["eps"]),
                   float(cfg["theta"]), KV_DTYPES[kv_dtype])
        h = VP()
        _check(_lib.mth_decoder_create(C.byref(c), C.byref(h)))
        self._h = h
        self._dev = {}          # device copies of the weights (kept alive here)
        self.batch = 0
        self.prompt_len = 0

    def close(self):
        if getattr(self, "_h", None):
            _lib.mth_decoder_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def _up(self, key, a):
        torch = mythos_oil._torch()
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            a = a.view(np.int16)
        t = torch.from_numpy(a).to(self.device)
        self._dev[key] = t
        return t.data_ptr()

    def load(self, model: dict):
        """Upload a synth.decoder_model-layout model (numpy) and bind it."""
        cfg = self.cfg
        F, H = cfg["ffn"], cfg["hidden"]
        for i, ly in enumerate(model["layers"]):
            p = {k: self._up((i, k), ly[k]) for k in ("attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "cbq", "cbk",
                                                      "cbv", "cbo", "wgate_up", "cbgate_up", "wdown")}
            ncb = len(ly["cbgate_up"]) // 2
            w = Layer(p["attn_norm"], p["ffn_norm"], p["wq"], p["wk"], p["wv"], p["wo"], p["cbq"], p["cbk"],
                      p["cbv"], p["cbo"], p["wgate_up"], p["wgate_up"] + F * (H // 2), p["cbgate_up"],
                      p["cbgate_up"] + ncb * 2, p["wdown"], float(ly["down_scale"]))
            _check(_lib.mth_decoder_set_layer(self._h, i, C.byref(w)))
        g = Globals(*[self._up(k, model[k]) for k in ("emb", "final_norm", "lm_idx", "lm_cb")])
        _check(_lib.mth_decoder_set_globals(self._h, C.byref(g)))

    def start(self, prompts: np.ndarray, stream=None):
        torch = mythos_oil._torch()
        prompts = np.ascontiguousarray(prompts, np.int32)
        if prompts.ndim == 1:
            prompts = prompts[None]
        self._prompts = torch.from_numpy(prompts).to(self.device)
        self.batch, self.prompt_len = prompts.shape
        _check(_lib.mth_decoder_start(self._h, self._prompts.data_ptr(), self.batch, self.prompt_len,
                                      mythos_oil._stream(stream)))

    def step(self, n: int = 1, graph: bool = True, stream=None):
        _check(_lib.mth_decoder_step(self._h, n, int(graph), mythos_oil._stream(stream)))

    def prefill(self, stream=None):
        """The prompt as one forward pass (mth_decoder_prefill): afterwards
        as after prompt_len steps."""
        _check(_lib.mth_decoder_prefill(self._h, mythos_oil._stream(stream)))

    @property
    def steps_done(self) -> int:
        return int(_lib.mth_decoder_steps_done(self._h))

    @property
    def launches_per_step(self) -> int:
        """Kernel launches of one graph step (0 before the first graph step)."""
        return int(_lib.mth_decoder_launches(self._h))

    def _buffers(self):
        lg, hist, stride = VP(), VP(), I64()
        _check(_lib.mth_decoder_buffers(self._h, C.byref(lg), C.byref(hist), C.byref(stride)))
        return lg.value, hist.value, stride.value

    def logits(self, stream=None) -> np.ndarray:
        """Logits [batch][vocab] of the last step (host copy; synchronises)."""
        out = np.empty((self.batch, self.cfg["vocab"]), np.float32)
        _check(_lib.mth_decoder_read(self._h, out.ctypes.data, None, mythos_oil._stream(stream)))
        return out

    def tokens(self, stream=None) -> np.ndarray:
        """Token history [batch][prompt_len + generated] (host copy)."""
        _, _, stride = self._buffers()
        out = np.empty((self.batch, stride), np.int32)
        _check(_lib.mth_decoder_read(self._h, None, out.ctypes.data, mythos_oil._stream(stream)))
        n = min(stride, max(self.prompt_len, self.steps_done + 1))
        return out[:, :n]

    def enable_taps(self):
        """Turn on the per-layer taps (mth_decoder_set_taps) for the started
        batch; later steps run without a graph."""
        torch = mythos_oil._torch()
        n = int(_lib.mth_decoder_tap_floats(self._h))
        self._taps = torch.zeros(self.cfg["layers"] * n, dtype=torch.float32, device=self.device)
        _check(_lib.mth_decoder_set_taps(self._h, self._taps.data_ptr()))

    def disable_taps(self):
        _check(_lib.mth_decoder_set_taps(self._h, None))
        self._taps = None

    def taps(self) -> list:
        """Host copies of the last step's taps: one dict per layer with
        x_attn [B][H], gate [B][F], up [B][F], act [B][F], aq [B][F] int8,
        a_inv [B], down [B][H]."""
        torch = mythos_oil._torch()
        torch.cuda.synchronize()
        B, H, F = self.batch, self.cfg["hidden"], self.cfg["ffn"]
        n = int(_lib.mth_decoder_tap_floats(self._h))
        t = self._taps.cpu().numpy().reshape(self.cfg["layers"], n)
        out = []
        for row in t:
            o, d = 0, {}
            for name, size in (("x_attn", B * H), ("gu", B * 2 * F), ("act", B * F), ("aq", B * F // 4),
                               ("a_inv", B), ("down", B * H)):
                d[name] = row[o:o + size]
                o += size
            gu = d.pop("gu").reshape(B, 2 * F)
            d["gate"], d["up"] = gu[:, :F].copy(), gu[:, F:].copy()
            d["x_attn"] = d["x_attn"].reshape(B, H)
            d["act"] = d["act"].reshape(B, F)
            d["aq"] = np.ascontiguousarray(d["aq"]).view(np.int8).reshape(B, F)
            d["down"] = d["down"].reshape(B, H)
            out.append(d)
        return out

    def read_kv(self, layer: int, stream=None):
        """Layer `layer`'s K and V caches as FP32 host arrays
        [batch][kv_heads][max_seq][head_dim] (bf16 caches widened exactly)."""
        c = self.cfg
        shape = (self.batch, c["kv_heads"], c["max_seq"], c["head_dim"])
        dt = np.uint16 if self.kv_dtype == "bf16" else np.float32
        k, v = np.empty(shape, dt), np.empty(shape, dt)
        _check(_lib.mth_decoder_read_kv(self._h, layer, k.ctypes.data, v.ctypes.data, mythos_oil._stream(stream)))
        if dt == np.uint16:
            k, v = ((a.astype(np.uint32) << 16).view(np.float32) for a in (k, v))
        return k, v

    def generate(self, prompts: np.ndarray, max_tokens: int, graph: bool = True, prefill: bool = True) -> np.ndarray:
        """Generator::generate_tokens with greedy sampling and no EOS stop:
        prompt_len + max_tokens ids per sequence.  The prompt runs as one
        forward pass (prefill), or with prefill=False as prompt_len steps."""
        self.start(prompts)
        if prefill:
            self.prefill()
            self.step(max_tokens - 1, graph=graph)
        else:
            self.step(self.prompt_len + max_tokens - 1, graph=graph)
        return self.tokens()[:, :self.prompt_len + max_tokens]

