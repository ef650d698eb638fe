"""ctypes binding of include/rpg_text.h: the engine's text front-end (BBPE
tokenizer, Qwen3 ChatML rendering, reply parsing) on the host CPU, the same
code rpg_engine_generate runs (reference src/tokenizer.h, src/chat_template.h,
src/tool_parser.h)."""

from __future__ import annotations

import ctypes
import json

import numpy as np

from . import EngineError, lib  # noqa: F401  (EngineError: the errors raised here)

_P, _I32, _I64, _U32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
_SIGS = {
    "rpg_text_tokenizer_load": ([ctypes.c_char_p], _I32),
    "rpg_text_tokenizer_free": ([_I32], None),
    "rpg_text_vocab_size": ([_I32], _I32),
    "rpg_text_encode": ([_I32, ctypes.c_char_p, _I64, _I32, _P, _I64], _I64),
    "rpg_text_decode": ([_I32, _P, _I64, _I32, ctypes.POINTER(_I64)], _P),
    "rpg_text_split": ([_I32, ctypes.c_char_p, _I64, _P, _I64], _I64),
    "rpg_text_render_chatml": ([ctypes.c_char_p], _P),
    "rpg_text_parse_reply": ([ctypes.c_char_p, _I64], _P),
    "rpg_text_char_classes": ([_U32, _I64, _P], _I32),
    "rpg_text_json_redump": ([ctypes.c_char_p, _I32], _P),
}
_ready = False


def _lib():
    global _ready
    L = lib()
    if not _ready:
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name)
            f.argtypes, f.restype = args, res
        L.rpg_engine_free.argtypes = [_P]
        L.rpg_engine_last_error.restype = ctypes.c_char_p
        _ready = True
    return L


def _err():
    return EngineError(_lib().rpg_engine_last_error().decode("utf-8", "replace"))


def _take(ptr, n=None) -> bytes:
    """The bytes of a string the library returned, freed afterwards."""
    if not ptr:
        raise _err()
    try:
        return ctypes.string_at(ptr, n) if n is not None else ctypes.string_at(ptr)
    finally:
        _lib().rpg_engine_free(ptr)


def _b(text) -> bytes:
    return text.encode("utf-8") if isinstance(text, str) else bytes(text)


class Tokenizer:
    """The BBPE tokenizer of a GGUF (its tokenizer.ggml.* metadata)."""

    def __init__(self, gguf_path: str):
        self.h = _lib().rpg_text_tokenizer_load(gguf_path.encode())
        if self.h < 0:
            raise _err()

    def __len__(self) -> int:
        return int(_lib().rpg_text_vocab_size(self.h))

    def encode(self, text, parse_special: bool = True) -> np.ndarray:
        t = _b(text)
        n = _lib().rpg_text_encode(self.h, t, len(t), int(parse_special), None, 0)
        if n < 0:
            raise _err()
        out = np.empty(n, dtype=np.int32)
        _lib().rpg_text_encode(self.h, t, len(t), int(parse_special), out.ctypes.data, n)
        return out

    def decode(self, ids, skip_special: bool = False) -> bytes:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        n = _I64()
        p = _lib().rpg_text_decode(self.h, a.ctypes.data, a.size, int(skip_special), ctypes.byref(n))
        return _take(p, n.value) if p else _take(p)

    def split(self, text) -> list:
        """The pre-tokenizer's pieces (bytes)."""
        t = _b(text)
        n = _lib().rpg_text_split(self.h, t, len(t), None, 0)
        if n < 0:
            raise _err()
        lens = np.empty(n, dtype=np.int64)
        _lib().rpg_text_split(self.h, t, len(t), lens.ctypes.data, n)
        out, at = [], 0
        for k in lens:
            out.append(t[at:at + int(k)])
            at += int(k)
        return out

    def close(self):
        if getattr(self, "h", -1) >= 0:
            _lib().rpg_text_tokenizer_free(self.h)
            self.h = -1

    __del__ = close


def render_chatml(request) -> bytes:
    """The ChatML prompt of a request (dict or JSON text)."""
    req = request if isinstance(request, (str, bytes)) else json.dumps(request, ensure_ascii=False)
    return _take(_lib().rpg_text_render_chatml(_b(req)))


def parse_reply(text) -> bytes:
    """The parse of a decoded reply as compact JSON (bytes)."""
    t = _b(text)
    return _take(_lib().rpg_text_parse_reply(t, len(t)))


def char_classes(first: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    if _lib().rpg_text_char_classes(first, n, out.ctypes.data) != 0:
        raise _err()
    return out


def json_redump(text, python: bool) -> bytes:
    return _take(_lib().rpg_text_json_redump(_b(text), int(python)))
