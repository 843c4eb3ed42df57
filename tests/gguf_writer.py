"""A small GGUF v3 writer for the tests, from the public file format:
u32 magic "GGUF", u32 version, u64 tensor count, u64 key count, the keys
({string, u32 type, value}; arrays: u32 element type, u64 count, elements),
the tensor infos ({string name, u32 n_dims, u64 ne[], u32 ggml type, u64
offset}), padding to the alignment, and the tensor data.  Strings are a u64
length and the bytes; everything is little-endian."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 0, 1, 8, 12, 14, 30


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_SCALAR[t], v)


def write_gguf(path, kv: list, tensors: list, alignment: int = 32, version: int = 3, magic: bytes = b"GGUF"):
    """kv: [(key, type, value)]; tensors: [(name, ggml type, ne list, bytes)]."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kv))
    meta = b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kv)
    infos, blobs, off = [], [], 0
    for name, gtype, ne, data in tensors:
        data = bytes(data)
        infos.append(_str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
                     + struct.pack("<IQ", gtype, off))
        pad = (-len(data)) % alignment
        blobs.append(data + b"\0" * pad)
        off += len(data) + pad
    body = head + meta + b"".join(infos)
    body += b"\0" * ((-len(body)) % alignment)
    with open(path, "wb") as f:
        f.write(body + b"".join(blobs))


def bf16(a: np.ndarray) -> bytes:
    """Round-to-nearest-even bf16 of an f32 array."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r.tobytes()


def bf16_round(a: np.ndarray) -> np.ndarray:
    """The f32 values a bf16 tensor written by bf16() reads back as."""
    return (np.frombuffer(bf16(a), np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(np.shape(a))


def write_layers(path, shape, layers: dict, arch: str, router_types=None, eps: float = 1e-6):
    """A GGUF holding the expert stage of `layers` ({index: HostLayer}) in the
    tensor names and shapes llama.cpp writes for MoE models.  router_types maps a
    layer to GGML_F32 / GGML_F16 / GGML_BF16 for its ffn_gate_inp (default f32);
    ffn_gate_inp_shexp is written as bf16.  Returns {index: (router, sh_gate_inp)}
    as the file holds them, in f32."""
    kv = [("general.architecture", STRING, arch), ("general.alignment", U32, 32),
          (f"{arch}.block_count", U32, len(layers)), (f"{arch}.embedding_length", U32, shape.n_embd),
          (f"{arch}.expert_feed_forward_length", U32, shape.n_ff), (f"{arch}.expert_count", U32, shape.n_expert),
          (f"{arch}.expert_used_count", U32, shape.n_used),
          (f"{arch}.attention.layer_norm_rms_epsilon", F32, eps)]
    if shape.n_ff_shexp:
        kv.append((f"{arch}.expert_shared_feed_forward_length", U32, shape.n_ff_shexp))
    E, D, F = shape.n_expert, shape.n_embd, shape.n_ff
    tensors, held = [], {}
    for l in sorted(layers):
        hl = layers[l]
        rt = (router_types or {}).get(l, GGML_F32)
        r = np.asarray(hl.router, np.float32).reshape(E, D)
        if rt == GGML_F32:
            rb, rf = r.tobytes(), r
        elif rt == GGML_F16:
            rb, rf = r.astype(np.float16).tobytes(), r.astype(np.float16).astype(np.float32)
        else:
            rb, rf = bf16(r), bf16_round(r)
        ls = hl.shape  # per-layer quant types, as in Q4_K_M files
        tensors += [(f"blk.{l}.ffn_gate_inp.weight", rt, [D, E], rb),
                    (f"blk.{l}.ffn_gate_exps.weight", ls.gate_type, [D, F, E], hl.gate.tobytes()),
                    (f"blk.{l}.ffn_up_exps.weight", ls.up_type, [D, F, E], hl.up.tobytes()),
                    (f"blk.{l}.ffn_down_exps.weight", ls.down_type, [F, D, E], hl.down.tobytes())]
        gi = None
        if shape.n_ff_shexp:
            S = shape.n_ff_shexp
            gi = bf16_round(hl.sh_gate_inp)
            tensors += [(f"blk.{l}.ffn_gate_shexp.weight", ls.sh_gate_type, [D, S], hl.sh_gate.tobytes()),
                        (f"blk.{l}.ffn_up_shexp.weight", ls.sh_up_type, [D, S], hl.sh_up.tobytes()),
                        (f"blk.{l}.ffn_down_shexp.weight", ls.sh_down_type, [S, D], hl.sh_down.tobytes()),
                        (f"blk.{l}.ffn_gate_inp_shexp.weight", GGML_BF16, [D], bf16(hl.sh_gate_inp))]
        held[l] = (rf.ravel(), gi)
    write_gguf(path, kv, tensors)
    return held


def write_stage_streaming(path, shape, n_layer: int, make_layer, arch: str, eps: float = 1e-6,
                          alignment: int = 32):
    """The expert stage of n_layer layers, layer by layer: make_layer(l) returns
    layer l's HostLayer (same quant types in every layer), which is written and
    dropped before the next is made.  f32 routers, bf16 shared gate rows."""
    import os
    from hoard_amd import expert_bytes
    D, F, E, S = shape.n_embd, shape.n_ff, shape.n_expert, shape.n_ff_shexp
    kv = [("general.architecture", STRING, arch), ("general.alignment", U32, alignment),
          (f"{arch}.block_count", U32, n_layer), (f"{arch}.embedding_length", U32, D),
          (f"{arch}.expert_feed_forward_length", U32, F), (f"{arch}.expert_count", U32, E),
          (f"{arch}.expert_used_count", U32, shape.n_used),
          (f"{arch}.attention.layer_norm_rms_epsilon", F32, eps)]
    if S:
        kv.append((f"{arch}.expert_shared_feed_forward_length", U32, S))
    per_layer = [("ffn_gate_inp", GGML_F32, [D, E], 4 * D * E),
                 ("ffn_gate_exps", shape.gate_type, [D, F, E], E * expert_bytes(shape.gate_type, F, D)),
                 ("ffn_up_exps", shape.up_type, [D, F, E], E * expert_bytes(shape.up_type, F, D)),
                 ("ffn_down_exps", shape.down_type, [F, D, E], E * expert_bytes(shape.down_type, D, F))]
    if S:
        per_layer += [("ffn_gate_shexp", shape.sh_gate_type, [D, S], expert_bytes(shape.sh_gate_type, S, D)),
                      ("ffn_up_shexp", shape.sh_up_type, [D, S], expert_bytes(shape.sh_up_type, S, D)),
                      ("ffn_down_shexp", shape.sh_down_type, [S, D], expert_bytes(shape.sh_down_type, D, S)),
                      ("ffn_gate_inp_shexp", GGML_BF16, [D], 2 * D)]
    infos, off = [], 0
    for l in range(n_layer):
        for name, t, ne, nb in per_layer:
            infos.append(_str(f"blk.{l}.{name}.weight") + struct.pack("<I", len(ne))
                         + b"".join(struct.pack("<Q", d) for d in ne) + struct.pack("<IQ", t, off))
            off += nb + (-nb) % alignment
    head = b"GGUF" + struct.pack("<IQQ", 3, len(infos), len(kv))
    head += b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kv) + b"".join(infos)
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        for l in range(n_layer):
            hl = make_layer(l)
            blobs = [np.asarray(hl.router, np.float32).tobytes(), hl.gate, hl.up, hl.down]
            if S:
                blobs += [hl.sh_gate, hl.sh_up, hl.sh_down, bf16(hl.sh_gate_inp)]
            for b, (_, _, _, nb) in zip(blobs, per_layer):
                mv = memoryview(b).cast("B") if not isinstance(b, bytes) else b
                assert len(mv) == nb
                f.write(mv)
                f.write(b"\0" * ((-nb) % alignment))
        f.flush()
        os.fsync(f.fileno())
