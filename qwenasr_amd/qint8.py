"""Host mirror of the reference's .qint8 reader over the C-ABI.

``QuantFile`` follows ``QuantFile`` (crates/qwen-asr/src/quantize.rs:108-330):
``open`` returns ``None`` where the reference's does (missing file, bad magic,
a name that is not UTF-8), ``find``/``has_tensor``/``is_self_contained`` have
the same meaning, and the getters hand out device tensors instead of pointers
into the mapping: ``get_quant_weight`` (quantize.rs:252-268) an int8
[out_dim, in_dim] matrix with its row scales, ``get_f32`` (quantize.rs:272-
305) an f32 tensor for F32 and BF16 entries, ``get_bf16_direct``
(quantize.rs:309-315) the raw bf16 bits. ``fused_gate_up`` builds the
interleaved gate/up matrix of ``DecoderInt8::load`` (decoder.rs:697-719)
directly in device memory. ``load_decoder_int8`` gathers the per-layer decoder
weight set ``DecoderInt8::load`` reads (decoder.rs:675-745) and
``detect_decoder_dims`` the decoder sizes ``QwenConfig::detect`` takes from
the table (config.rs:110-160, context.rs:359-373).

Every byte goes through libqasr_hip.so (parse and host-to-device copy); the
only torch work is allocating the destinations.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from . import kernels as K
from .kernels import QuantWeight

INT8, F32, BF16 = 0, 1, 2
VOCAB_SIZE = 151936  # config.rs:7


@dataclass
class QuantTensorMeta:
    """quantize.rs:51-72."""

    name: str
    dtype: int
    shape: tuple
    data_offset: int
    scale_offset: int

    @property
    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def out_dim(self) -> int:
        return self.shape[0] if self.shape else 0

    @property
    def in_dim(self) -> int:
        if len(self.shape) < 2:
            return 0
        n = 1
        for d in self.shape[1:]:
            n *= d
        return n


def _stream_ptr() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class QuantFile:
    """An open .qint8 file (read-only mapping held until ``close``)."""

    def __init__(self, handle: ctypes.c_void_p):
        self._h = handle
        ver = ctypes.c_int()
        n = ctypes.c_size_t()
        _lib.call("qasr_qint8_info", self._h, ctypes.byref(ver), ctypes.byref(n))
        self.version = ver.value
        self.tensors: list[QuantTensorMeta] = []
        self._index: dict[str, int] = {}
        name = ctypes.c_char_p()
        name_len, dtype, n_dims = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_size_t()
        shape = (ctypes.c_uint64 * 256)()
        doff, soff = ctypes.c_uint64(), ctypes.c_uint64()
        for i in range(n.value):
            _lib.call("qasr_qint8_tensor", self._h, i, ctypes.byref(name), ctypes.byref(name_len),
                      ctypes.byref(dtype), ctypes.byref(n_dims), shape, 256, ctypes.byref(doff),
                      ctypes.byref(soff))
            nm = ctypes.string_at(ctypes.cast(name, ctypes.c_void_p), name_len.value).decode()
            self.tensors.append(QuantTensorMeta(nm, dtype.value, tuple(shape[:n_dims.value]),
                                                doff.value, soff.value))
            self._index[nm] = i  # a repeated name maps to its last entry, as in the C table

    @classmethod
    def open(cls, path: str) -> "QuantFile | None":
        """QuantFile::open: ``None`` for a missing or malformed file."""
        h = ctypes.c_void_p()
        rc = _lib.lib().qasr_qint8_open(str(path).encode(), ctypes.byref(h))
        if rc != _lib.QASR_OK:
            return None
        return cls(h)

    def close(self) -> None:
        if self._h:
            h, self._h = self._h, None
            _lib.call("qasr_qint8_close", h)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # --- lookup ---------------------------------------------------------
    def find(self, name: str) -> QuantTensorMeta | None:
        i = self._index.get(name)
        return None if i is None else self.tensors[i]

    def has_tensor(self, name: str) -> bool:
        return name in self._index

    def is_self_contained(self) -> bool:
        """quantize.rs:323-325: a V2 file that also holds the audio encoder."""
        return self.has_tensor("thinker.audio_tower.layers.0.self_attn.q_proj.weight")

    # --- device uploads --------------------------------------------------
    def _upload(self, i: int, data: torch.Tensor, scales: torch.Tensor | None) -> None:
        _lib.call("qasr_qint8_upload", self._h, i, ctypes.c_void_p(data.data_ptr()),
                  ctypes.c_void_p(scales.data_ptr() if scales is not None else 0), _stream_ptr())

    def get_quant_weight(self, name: str, device="cuda") -> QuantWeight | None:
        """Device copy of an INT8 entry (quantize.rs:259-273). The reference
        returns a view for any dtype, reading an F32/BF16 entry's bytes as int8
        with a scale pointer at offset 0; this mirror raises ``ValueError`` for
        those entries instead of uploading bytes that are not int8 weights."""
        m = self.find(name)
        if m is None:
            return None
        if m.dtype != INT8:
            raise ValueError(f"{name} is not an INT8 tensor")
        if len(m.shape) < 2:
            raise ValueError(f"{name}: an INT8 weight has at least two dimensions, got {m.shape}")
        data = torch.empty((m.out_dim, m.in_dim), dtype=torch.int8, device=device)
        scales = torch.empty(m.out_dim, dtype=torch.float32, device=device)
        self._upload(self._index[name], data, scales)
        return QuantWeight(data, scales, m.out_dim, m.in_dim)

    def get_bf16_direct(self, name: str, device="cuda") -> torch.Tensor | None:
        m = self.find(name)
        if m is None or m.dtype != BF16:
            return None
        out = torch.empty(m.shape, dtype=torch.bfloat16, device=device)
        self._upload(self._index[name], out, None)
        return out

    def get_f32(self, name: str, device="cuda") -> torch.Tensor | None:
        """quantize.rs:276-306: F32 entries as stored; BF16 entries widened to
        f32 (exact); INT8 entries dequantized, ``f32[o, k] = int8[o, k] * scale[o]``
        (one f32 multiply per element, done by the int8 row-gather kernel over
        every row, which is exactly that product)."""
        m = self.find(name)
        if m is None:
            return None
        if m.dtype == F32:
            out = torch.empty(m.shape, dtype=torch.float32, device=device)
            self._upload(self._index[name], out, None)
            return out
        if m.dtype == BF16:
            return self.get_bf16_direct(name, device).float()
        w = self.get_quant_weight(name, device)
        out = torch.empty((w.out_dim, w.in_dim), dtype=torch.float32, device=device)
        if w.out_dim and w.in_dim:
            rows = torch.arange(w.out_dim, dtype=torch.int32, device=device)
            K.embed_gather_i8(out, w, rows, w.out_dim, w.in_dim)
        return out.reshape(m.shape)

    def fused_gate_up(self, gate_name: str, up_name: str, inter: int, hidden: int,
                      device="cuda") -> QuantWeight:
        w = torch.empty((2 * inter, hidden), dtype=torch.int8, device=device)
        s = torch.empty(2 * inter, dtype=torch.float32, device=device)
        _lib.call("qasr_qint8_upload_gate_up", self._h, gate_name.encode(), up_name.encode(),
                  inter, hidden, ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(s.data_ptr()),
                  _stream_ptr())
        return QuantWeight(w, s, 2 * inter, hidden)


@dataclass
class DecoderDims:
    hidden: int
    intermediate: int
    lm_head_dim: int
    n_layers: int = 28  # config.rs:70 default
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128


def detect_decoder_dims(qf: QuantFile) -> DecoderDims:
    """The decoder fields of QwenConfig::detect on a .qint8 table."""
    emb = qf.find("thinker.model.embed_tokens.weight")
    gate = qf.find("thinker.model.layers.0.mlp.gate_proj.weight")
    lm = qf.find("thinker.lm_head.weight")
    big_enc = qf.has_tensor("thinker.audio_tower.layers.18.self_attn.q_proj.weight")
    hidden = emb.shape[1] if emb is not None and len(emb.shape) == 2 else (2048 if big_enc else 1024)
    inter = gate.shape[0] if gate is not None and len(gate.shape) == 2 else (
        6144 if hidden >= 2048 else 3072)
    lm_dim = VOCAB_SIZE
    if lm is not None and len(lm.shape) == 2 and lm.shape[0] != VOCAB_SIZE:
        lm_dim = lm.shape[0]  # forced aligner classify_num
    return DecoderDims(hidden, inter, lm_dim)


def load_decoder_int8(qf: QuantFile, dims: DecoderDims, device="cuda") -> dict | None:
    """Device copy of the weights DecoderInt8::load reads; ``None`` if one is missing."""
    out = {"tok_embeddings": qf.get_quant_weight("thinker.model.embed_tokens.weight", device)}
    if out["tok_embeddings"] is None:
        return None
    layers = []
    for i in range(dims.n_layers):
        lp = f"thinker.model.layers.{i}"
        names = {k: f"{lp}.self_attn.{k}_proj.weight" for k in ("q", "k", "v", "o")}
        names.update(gate=f"{lp}.mlp.gate_proj.weight", up=f"{lp}.mlp.up_proj.weight",
                     down=f"{lp}.mlp.down_proj.weight")
        norms = {"q_norm": f"{lp}.self_attn.q_norm.weight", "k_norm": f"{lp}.self_attn.k_norm.weight",
                 "input_norm": f"{lp}.input_layernorm.weight",
                 "post_attn_norm": f"{lp}.post_attention_layernorm.weight"}
        if not all(qf.has_tensor(n) for n in list(names.values()) + list(norms.values())):
            return None
        layer = {f"w{k}": qf.get_quant_weight(names[k], device) for k in ("q", "k", "v", "o")}
        layer.update({k: qf.get_f32(v, device) for k, v in norms.items()})
        layer["gate_up"] = qf.fused_gate_up(names["gate"], names["up"], dims.intermediate,
                                            dims.hidden, device)
        layer["down"] = qf.get_quant_weight(names["down"], device)
        layers.append(layer)
    out["layers"] = layers
    out["norm"] = qf.get_f32("thinker.model.norm.weight", device)
    if out["norm"] is None:
        return None
    out["lm_head"] = qf.get_quant_weight("thinker.lm_head.weight", device)  # optional (tied)
    return out
