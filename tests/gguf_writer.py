"""Minimal GGUF v3 writer for the tests (TEST INFRASTRUCTURE).

Writes the container the engine loads (src/gguf.c:104-283): the "GGUF"
magic, version 3, tensor and metadata counts, metadata key/value pairs, the
tensor table (name, dims with ne0 fastest, GGML type, offset relative to the
data section) and the data section starting at the next multiple of the
alignment, each tensor's offset aligned too.  The tensors' bytes are whatever
the caller passes: here the CPU oracle's own Q4_K / Q6_K quantisations, so a
GPU run on the loaded tensors can be checked against the oracle on the same
bytes.
"""
from __future__ import annotations

import struct

import numpy as np

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
# GGML tensor types used here
T_F32, T_F16, T_Q4_K, T_Q6_K = 0, 1, 12, 14
BLOCK = {T_F32: (1, 4), T_F16: (1, 2), T_Q4_K: (256, 144), T_Q6_K: (256, 210)}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t: int, v) -> bytes:
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    return struct.pack(fmt[t], v)


def tensor_bytes(ttype: int, dims) -> int:
    blk, bs = BLOCK[ttype]
    n = 1
    for d in dims[1:]:
        n *= d
    return dims[0] // blk * bs * n


def write_gguf(path, metadata, tensors, alignment: int = 32, version: int = 3):
    """metadata: [(key, type, value)]; tensors: [(name, ggml_type, dims, bytes)]
    with dims ne0-first.  A general.alignment entry, if wanted, is the
    caller's to include (the reader uses it)."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata))
    kv = b"".join(_str(k) + struct.pack("<I", t) + _val(t, v) for k, t, v in metadata)
    infos = []
    off = 0
    for name, ttype, dims, data in tensors:
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        infos.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) +
                     struct.pack("<IQ", ttype, off))
        off += (data.size + alignment - 1) // alignment * alignment
    table = head + kv + b"".join(infos)
    pad = (-len(table)) % alignment
    with open(path, "wb") as f:
        f.write(table + b"\0" * pad)
        for name, ttype, dims, data in tensors:
            data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            f.write(data.tobytes())
            f.write(b"\0" * ((-data.size) % alignment))


def moe_model_tensors(layers, prefix: str = "blk"):
    """The MoE FFN tensors of host layers (oracle HostLayer objects) under the
    names and shapes the engine resolves (gguf.c:318-326): router
    [n_embd, n_expert] f32, expert gate/up [n_embd, n_ff, n_expert], down
    [n_ff, n_embd, n_expert], shared gate [n_embd] f32, shared gate/up
    [n_embd, n_ff], shared down [n_ff, n_embd]."""
    out = []
    for il, L in enumerate(layers):
        N, F, E = L.n_embd, L.n_ff, L.n_expert
        p = f"{prefix}.{il}."
        out += [
            (p + "ffn_gate_inp.weight", T_F32, [N, E], L.gate_inp),
            (p + "ffn_gate_exps.weight", T_Q4_K, [N, F, E], L.gate_exps),
            (p + "ffn_up_exps.weight", T_Q4_K, [N, F, E], L.up_exps),
            (p + "ffn_down_exps.weight", L.t_down_exps, [F, N, E], L.down_exps),
            (p + "ffn_gate_inp_shexp.weight", T_F32, [N], L.gate_inp_shexp),
            (p + "ffn_gate_shexp.weight", T_Q4_K, [N, F], L.gate_shexp),
            (p + "ffn_up_shexp.weight", T_Q4_K, [N, F], L.up_shexp),
            (p + "ffn_down_shexp.weight", L.t_down_shexp, [F, N], L.down_shexp),
        ]
    return out


def qwen35moe_metadata(n_layer: int, n_embd: int, n_expert: int, n_used: int, n_ff: int):
    """Metadata a qwen35moe GGUF carries for this path, plus entries of every
    other value kind (strings, arrays, floats, bools) the reader must skip."""
    return [
        ("general.architecture", STR, "qwen35moe"),
        ("general.name", STR, "synthetic qwen35moe FFN stack"),
        ("qwen35moe.block_count", U32, n_layer),
        ("qwen35moe.embedding_length", U32, n_embd),
        ("qwen35moe.expert_count", U32, n_expert),
        ("qwen35moe.expert_used_count", U32, n_used),
        ("qwen35moe.expert_feed_forward_length", U32, n_ff),
        ("qwen35moe.expert_shared_feed_forward_length", U32, n_ff),
        ("qwen35moe.rope.freq_base", F32, 1e7),
        ("qwen35moe.rope.dimension_sections", ARR, (I32, [11, 11, 10, 0])),
        ("tokenizer.ggml.tokens", ARR, (STR, ["<a>", "b", "cd", "é", ""])),
        ("tokenizer.ggml.add_bos_token", BOOL, False),
        ("general.sampling.temp", F64, 0.7),
    ]
