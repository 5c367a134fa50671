"""Synthetic GGUF files for the format tests (no GGUF file ships with the
reference; its own loader tests build theirs in memory the same way,
gguf_loader.rs:4382-4450, :4960-5000).

Layout written (GGUF v1-v3): "GGUF", u32 version, tensor count and KV
count (u32 in v1, u64 after), KV pairs (string key, u32 type, value),
tensor infos (string name, u32 n_dims, dims (u32 in v1, u64 after), u32
ggml type, u64 data offset), zero padding to general.alignment (default
32), tensor data.  Strings are a length (u32 in v1, u64 after) + bytes.
"""
from __future__ import annotations

import struct

import numpy as np

GGML_F32, GGML_Q4_0, GGML_Q8_0 = 0, 2, 8
BLOCK = {GGML_Q4_0: (32, 18), GGML_Q8_0: (32, 34), GGML_F32: (1, 4)}

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q",
        F64: "<d"}


def _count(version, n):
    return struct.pack("<I" if version == 1 else "<Q", n)


def _string(version, s):
    b = s.encode()
    return _count(version, len(b)) + b


def _value(version, ty, v):
    if ty == STRING:
        return _string(version, v)
    if ty == ARRAY:
        et, items = v
        return struct.pack("<I", et) + _count(version, len(items)) + b"".join(_value(version, et, x) for x in items)
    return struct.pack(_FMT[ty], v)


def tensor_bytes(ggml_type, dims):
    n = int(np.prod(dims))
    elems, nbytes = BLOCK[ggml_type]
    assert n % elems == 0
    return n // elems * nbytes


def write_gguf(path, kv, tensors, version=3, alignment=None):
    """kv: list of (key, type, value); tensors: list of (name, dims
    (GGML order, innermost first), ggml type, bytes).  Returns the offset
    of the tensor data section."""
    if alignment is not None:
        kv = list(kv) + [("general.alignment", U32, alignment)]
    align = alignment or 32
    head = b"GGUF" + struct.pack("<I", version) + _count(version, len(tensors)) + _count(version, len(kv))
    for key, ty, v in kv:
        head += _string(version, key) + struct.pack("<I", ty) + _value(version, ty, v)
    off, infos, body = 0, b"", b""
    for name, dims, ty, data in tensors:
        assert len(data) == tensor_bytes(ty, dims), name
        infos += _string(version, name) + struct.pack("<I", len(dims))
        infos += b"".join(struct.pack("<I" if version == 1 else "<Q", d) for d in dims)
        infos += struct.pack("<I", ty) + struct.pack("<Q", off)
        pad = (-len(data)) % align
        body += bytes(data) + b"\0" * pad
        off += len(data) + pad
    head += infos
    start = (len(head) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(head + b"\0" * (start - len(head)) + body)
    return start


def q_blocks(ggml_type, n_blocks, rng, scale=0.01):
    """n_blocks well-formed Q4_0 / Q8_0 blocks: f16 scale then quants."""
    d = (rng.random(n_blocks) * scale + scale * 0.1).astype(np.float16)
    if ggml_type == GGML_Q4_0:
        q = rng.integers(0, 256, size=(n_blocks, 16), dtype=np.uint8)
    else:
        q = rng.integers(-127, 128, size=(n_blocks, 32)).astype(np.int8).view(np.uint8)
    return np.concatenate([d.view(np.uint8).reshape(n_blocks, 2), q], axis=1).reshape(-1)


def moe_model(path, ggml_type, d_model, d_ff, n_experts, layers=(0,), per_expert=False, version=3, alignment=None,
              arch="mixtral", meta=None, seed=0):
    """A GGUF holding MoE expert tensors for `layers`.  Returns
    {layer: [(gate, up, down) bytes of each expert]} for checking."""
    rng = np.random.default_rng(seed)
    proj_blocks = d_model * d_ff // 32
    kv = [("general.architecture", STRING, arch)]
    if meta is None:
        meta = {f"{arch}.embedding_length": d_model, f"{arch}.expert_feed_forward_length": d_ff,
                f"{arch}.expert_count": n_experts}
    kv += [(k, U32, v) for k, v in meta.items()]
    kv += [("general.name", STRING, "synthetic"), ("tokenizer.ggml.scores", ARRAY, (F32, [0.5, 0.25, 0.125]))]
    tensors, expect = [], {}
    for layer in layers:
        parts = [[q_blocks(ggml_type, proj_blocks, rng) for _ in range(3)] for _ in range(n_experts)]
        expect[layer] = [tuple(p.tobytes() for p in e) for e in parts]
        dims = [[d_model, d_ff], [d_model, d_ff], [d_ff, d_model]]
        names = ["gate", "up", "down"]
        if per_expert:
            for e in range(n_experts):
                for i in range(3):
                    tensors.append((f"blk.{layer}.ffn_{names[i]}.{e}.weight", dims[i], ggml_type, parts[e][i]))
        else:
            for i in range(3):
                data = np.concatenate([parts[e][i] for e in range(n_experts)])
                tensors.append((f"blk.{layer}.ffn_{names[i]}_exps.weight", dims[i] + [n_experts], ggml_type, data))
        # a dense neighbour tensor, as real files hold
        tensors.append((f"blk.{layer}.attn_norm.weight", [d_model], GGML_F32, np.ones(d_model, np.float32).view(np.uint8)))
    write_gguf(path, kv, tensors, version=version, alignment=alignment)
    return expect
