"""GGUF v3 writer for synthetic models (the on-disk format GgufReader parses,
src/DotNetFoundryLLM.ModelFormats.Gguf/GgufReader.cs:37-93).

Layout: magic "GGUF", u32 version, u64 tensor count, u64 metadata count, metadata
(key string, u32 value type, value), tensor infos (name, u32 n_dims, u64 dims (innermost
first), u32 type, u64 offset relative to the data start), padding to `general.alignment`
(32), tensor data. Strings are u64 length + UTF-8 bytes.
"""
import os
import struct

import numpy as np

from . import _native as N
from .configs import ARCH_NAMES, synth_bytes, tensor_plan

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)


def _s(v):
    b = v.encode()
    return struct.pack("<Q", len(b)) + b


def _val(vtype, v):
    if vtype == STR:
        return _s(v)
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}[vtype]
    return struct.pack(fmt, v)


class GgufWriter:
    def __init__(self, path, alignment=32):
        self.path = path
        self.alignment = alignment
        self.meta = []
        self.tensors = []

    def add(self, key, vtype, value):
        self.meta.append((key, vtype, value))

    def add_array(self, key, etype, values):
        self.meta.append((key, ARR, (etype, list(values))))

    def add_tensor(self, name, dims, ttype, data, nbytes=None):
        """data: the tensor's bytes, or a callable returning them (then nbytes is required), so that
        a large file is written one tensor at a time."""
        if callable(data):
            self.tensors.append((name, list(dims), ttype, int(nbytes), data))
        else:
            a = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            self.tensors.append((name, list(dims), ttype, a.nbytes, lambda a=a: a))

    def write(self):
        out = bytearray()
        out += b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", len(self.tensors)) + struct.pack("<Q", len(self.meta))
        for key, vtype, value in self.meta:
            out += _s(key) + struct.pack("<I", vtype)
            if vtype == ARR:
                etype, vals = value
                out += struct.pack("<I", etype) + struct.pack("<Q", len(vals))
                for v in vals:
                    out += _val(etype, v)
            else:
                out += _val(vtype, value)
        offsets, off = [], 0
        for name, dims, ttype, nbytes, data in self.tensors:
            off = (off + self.alignment - 1) // self.alignment * self.alignment
            offsets.append(off)
            off += nbytes
        for (name, dims, ttype, nbytes, data), o in zip(self.tensors, offsets):
            out += _s(name) + struct.pack("<I", len(dims))
            for d in dims:
                out += struct.pack("<Q", d)
            out += struct.pack("<I", ttype) + struct.pack("<Q", o)
        pad = (len(out) + self.alignment - 1) // self.alignment * self.alignment - len(out)
        out += b"\0" * pad
        with open(self.path, "wb") as f:
            f.write(out)
            pos = 0
            for (name, dims, ttype, nbytes, data), o in zip(self.tensors, offsets):
                if o > pos:
                    f.write(b"\0" * (o - pos))
                a = np.ascontiguousarray(data()).view(np.uint8).reshape(-1)
                if a.nbytes != nbytes:
                    raise ValueError(f"{name}: {a.nbytes} bytes, declared {nbytes}")
                f.write(a.data)
                pos = o + nbytes
                del a


def write_synthetic_gguf(path, cfg, n_vocab_tokens=None):
    """Write cfg's seeded weights as a GGUF file the reference loader accepts: architecture keys
    under the arch prefix, a byte-encoder-safe token list (distinct printable ASCII strings) so
    the tokenizer builds, and no query_pre_attn_scalar (so Gemma2 uses 1/sqrt(head_dim))."""
    arch = ARCH_NAMES[cfg["arch"]]
    w = GgufWriter(path)
    w.add("general.architecture", STR, arch)
    w.add("general.name", STR, cfg["name"])
    w.add("general.alignment", U32, 32)
    w.add(f"{arch}.block_count", U32, cfg["n_layers"])
    w.add(f"{arch}.embedding_length", U32, cfg["hidden"])
    w.add(f"{arch}.feed_forward_length", U32, cfg["ffn"])
    w.add(f"{arch}.attention.head_count", U32, cfg["n_heads"])
    w.add(f"{arch}.attention.head_count_kv", U32, cfg["n_kv_heads"])
    w.add(f"{arch}.context_length", U32, cfg["max_ctx"])
    w.add(f"{arch}.vocab_size", U32, cfg["vocab"])
    w.add(f"{arch}.rope.freq_base", F32, cfg["rope_base"])
    if cfg["rope_scaled"]:
        w.add(f"{arch}.rope.scaling.type", STR, "linear")
        w.add(f"{arch}.rope.scaling.factor", F32, cfg["rope_scale"])
    if cfg["arch"] == N.ARCH_GEMMA2:
        w.add(f"{arch}.attention.key_length", U32, cfg["head_dim"])
        w.add(f"{arch}.attn_logit_softcapping", F32, cfg["attn_softcap"])
        w.add(f"{arch}.final_logit_softcapping", F32, cfg["final_softcap"])
    if cfg["window"] != 0x7FFFFFFF and cfg["arch"] in (N.ARCH_GEMMA2, N.ARCH_MISTRAL):
        w.add(f"{arch}.attention.sliding_window", U32, cfg["window"])
    nt = n_vocab_tokens or cfg["vocab"]
    w.add_array("tokenizer.ggml.tokens", STR, [f"t{i:x}" for i in range(nt)])
    w.add("tokenizer.ggml.bos_token_id", U32, 1)
    w.add("tokenizer.ggml.eos_token_id", U32, 2)
    for entry in tensor_plan(cfg):
        name, slot, layer, tt, rows, cols, dist, tid = entry
        n = rows * cols
        nbytes = n * {N.F32: 4, N.F16: 2, N.BF16: 2}[tt] if tt in (N.F32, N.F16, N.BF16) else N.type_bytes(tt, n)
        dims = [cols] if rows == 1 else [cols, rows]
        w.add_tensor(name, dims, tt, lambda e=entry: synth_bytes(cfg, e), nbytes)
    w.write()
    return path


def drop_page_cache(path):
    """Writes the file's dirty pages out and asks the kernel to drop its cached pages, so the next
    read of it comes from the disk (posix_fadvise DONTNEED on a file this process may read)."""
    fd = os.open(path, os.O_RDONLY)
    try:
        os.fsync(fd)
        os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
    finally:
        os.close(fd)
