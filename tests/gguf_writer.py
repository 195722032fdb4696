"""A GGUF v3 writer for the reader's tests, written from the GGUF v3
specification: header (magic, version, tensor and metadata counts),
metadata key/value pairs, tensor infos (name, dims, storage type, offset),
padding to the alignment, then the tensor data at aligned offsets.

It can also produce malformed files on purpose (raw field overrides) so the
reader's rejections are exercised.  Test infrastructure only."""
from __future__ import annotations

import struct

import numpy as np

# Metadata value types of the specification.
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}


def gguf_string(s: bytes | str) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def value_bytes(vtype: int, value) -> bytes:
    if vtype == STRING:
        return gguf_string(value)
    if vtype == ARRAY:
        etype, items = value
        return struct.pack("<IQ", etype, len(items)) + b"".join(value_bytes(etype, v) for v in items)
    return struct.pack(_SCALAR[vtype], value)


class GGUFWriter:
    def __init__(self, alignment: int | None = None, version: int = 3, magic: bytes = b"GGUF"):
        """alignment: the general.alignment written (None: key absent, 32
        applies); a value that is not a power of two is written as is and the
        data laid out at 32."""
        self.meta: list[bytes] = []
        self.tensors: list[dict] = []
        self.version = version
        self.magic = magic
        valid = alignment is not None and alignment > 0 and alignment & (alignment - 1) == 0
        self.alignment = alignment if valid else 32
        if alignment is not None:
            self.add("general.alignment", U32, alignment)

    def add(self, key: str, vtype: int, value) -> None:
        self.meta.append(gguf_string(key) + struct.pack("<I", vtype) + value_bytes(vtype, value))

    def add_raw_meta(self, raw: bytes) -> None:
        """A pre-encoded key/value entry (for malformed files)."""
        self.meta.append(raw)

    def add_tensor(self, name: str, dims, ttype: int, data: bytes, offset: int | None = None) -> None:
        self.tensors.append(dict(name=name, dims=list(dims), type=ttype, data=bytes(data), offset=offset))

    def to_bytes(self, n_tensors: int | None = None, n_meta: int | None = None) -> bytes:
        a = self.alignment
        # Offsets: consecutive, each aligned, unless a test fixes one.
        off = 0
        for t in self.tensors:
            if t["offset"] is None:
                off = (off + a - 1) // a * a
                t["_off"] = off
            else:
                t["_off"] = t["offset"]
            off = max(off, t["_off"] + len(t["data"]))
        head = self.magic + struct.pack("<IQQ", self.version,
                                        len(self.tensors) if n_tensors is None else n_tensors,
                                        len(self.meta) if n_meta is None else n_meta)
        head += b"".join(self.meta)
        for t in self.tensors:
            head += gguf_string(t["name"]) + struct.pack("<I", len(t["dims"]))
            head += b"".join(struct.pack("<Q", d) for d in t["dims"])
            head += struct.pack("<IQ", t["type"], t["_off"])
        data_start = (len(head) + a - 1) // a * a
        body = bytearray(off)
        for t in self.tensors:
            o = t["_off"]
            if o + len(t["data"]) <= len(body):
                body[o:o + len(t["data"])] = t["data"]
        return head + bytes(data_start - len(head)) + bytes(body)

    def write(self, path, **kw) -> bytes:
        b = self.to_bytes(**kw)
        with open(path, "wb") as f:
            f.write(b)
        return b


TENSOR_NAMES = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
                "up": "ffn_up", "down": "ffn_down"}


def llama_writer(cfg: dict, W: dict, tensor_shape, alignment: int | None = None, tokens=None,
                 vocab_size_key: bool = True, merges=None) -> GGUFWriter:
    """A Llama model in the tensor naming of the reference's lookups
    (inferencer.cu:1196-1214, 1434-1523): llama.* hyper-parameters, token
    embedding, output norm, optional output, and blk.N.* tensors with dims
    {cols, rows}."""
    w = GGUFWriter(alignment)
    w.add("general.architecture", STRING, "llama")
    w.add("llama.embedding_length", U32, cfg["dim"])
    w.add("llama.block_count", U32, cfg["layers"])
    w.add("llama.attention.head_count", U32, cfg["heads"])
    w.add("llama.attention.head_count_kv", U32, cfg["kv_heads"])
    w.add("llama.feed_forward_length", U32, cfg["hidden"])
    if vocab_size_key:
        w.add("llama.vocab_size", U32, cfg["vocab"])
    w.add("llama.attention.layer_norm_rms_epsilon", F32, cfg["eps"])
    w.add("llama.rope.freq_base", F32, cfg["rope_theta"])
    if tokens is not None:
        w.add("tokenizer.ggml.tokens", ARRAY, (STRING, tokens))
    if merges is not None:
        w.add("tokenizer.ggml.merges", ARRAY, (STRING, merges))
    dim = cfg["dim"]
    w.add_tensor("token_embd.weight", [dim, cfg["vocab"]], W["embd_type"], W["token_embd"].tobytes())
    w.add_tensor("output_norm.weight", [dim], 0, np.asarray(W["output_norm"], dtype=np.float32).tobytes())
    if W.get("output") is not None:
        w.add_tensor("output.weight", [dim, cfg["vocab"]], W["output_type"], W["output"].tobytes())
    for l, L in enumerate(W["layers"]):
        b = f"blk.{l}."
        w.add_tensor(b + "attn_norm.weight", [dim], 0, np.asarray(L["attn_norm"], dtype=np.float32).tobytes())
        w.add_tensor(b + "ffn_norm.weight", [dim], 0, np.asarray(L["ffn_norm"], dtype=np.float32).tobytes())
        for key, gname in TENSOR_NAMES.items():
            cols, rows = tensor_shape(cfg, key)
            w.add_tensor(b + gname + ".weight", [cols, rows], L[key + "_type"], L[key].tobytes())
    return w
