"""A small GGUF v3 writer and a tiny llama-architecture model built with it.

Test infrastructure: the file is what FISH's loader reads (`gguf.cpp:380-455`
for the container, `model.cpp:405-560` for the llama metadata and tensor
names, `tokenizer.cpp:160-250` for the SPM vocabulary). Weight bytes come from
`imurun_amd.quantize_rows`, whose bytes equal FISH's `quantize_row`.

GGUF v3 layout: magic "GGUF", version, tensor count, metadata count; the
metadata key/value pairs; one info record per tensor (name, dims with ne[0] the
row length, ggml type, offset into the data section); the data section,
aligned to `general.alignment` (32 here), with every tensor at an aligned
offset.
"""
from __future__ import annotations

import struct

import numpy as np

# GGUF metadata value types
U32, I32, F32, BOOL, STR, ARR, U64, F64 = 4, 5, 6, 7, 8, 9, 10, 12
ALIGN = 32


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind: int, v) -> bytes:
    if kind == U32:
        return struct.pack("<I", v)
    if kind == I32:
        return struct.pack("<i", v)
    if kind == F32:
        return struct.pack("<f", v)
    if kind == BOOL:
        return struct.pack("<B", 1 if v else 0)
    if kind == STR:
        return _str(v)
    if kind == U64:
        return struct.pack("<Q", v)
    if kind == F64:
        return struct.pack("<d", v)
    raise ValueError(kind)


def write_gguf(path: str, meta: list, tensors: list) -> None:
    """meta: (key, kind, value) with kind ARR taking (item_kind, items);
    tensors: (name, ne tuple, ggml type, bytes)."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for key, kind, v in meta:
        out += _str(key) + struct.pack("<I", kind)
        if kind == ARR:
            item_kind, items = v
            out += struct.pack("<IQ", item_kind, len(items))
            for it in items:
                out += _value(item_kind, it)
        else:
            out += _value(kind, v)
    offset = 0
    offsets = []
    for name, ne, t, data in tensors:
        offsets.append(offset)
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        out += struct.pack("<IQ", t, offset)
        offset += (len(data) + ALIGN - 1) // ALIGN * ALIGN
    out += bytes(-len(out) % ALIGN)
    base = len(out)
    for (name, ne, t, data), off in zip(tensors, offsets):
        out += bytes(base + off - len(out))
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(out)


# ---------------------------------------------------------------- tiny llama

def spm_vocab():
    """<unk>, <s>, </s>, the 256 byte tokens, then '▁' and the letters with and
    without the word-start mark; scores favour longer pieces."""
    toks = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    types = [2, 3, 3] + [6] * 256
    scores = [0.0, 0.0, 0.0] + [-1000.0] * 256
    for i, c in enumerate("abcdefghijklmnopqrstuvwxyz"):
        toks += [c, "▁" + c]
        types += [1, 1]
        scores += [-10.0 - i, -5.0 - i]
    toks.append("▁")
    types.append(1)
    scores.append(-50.0)
    return toks, scores, types


def tiny_llama(path: str, types: dict, seed: int = 7, n_layers: int = 2, n_embd: int = 256, n_ff: int = 768,
               n_head: int = 4, n_head_kv: int = 2, n_ctx: int = 512, raw=None) -> dict:
    """Writes a random llama model; `types` maps q, k, v, o, gate, up, down,
    output and embd to ggml type ids. Types without a block writer in
    imurun_amd take their bytes from raw(type, n_out, n_in, seed). Returns the
    configuration."""
    return tiny_model(path, types, seed=seed, n_layers=n_layers, n_embd=n_embd, n_ff=n_ff, n_head=n_head,
                      n_head_kv=n_head_kv, n_ctx=n_ctx, raw=raw)


def tiny_model(path: str, types: dict, arch: str = "llama", seed: int = 7, n_layers: int = 2, n_embd: int = 256,
               n_ff: int = 768, n_head: int = 4, n_head_kv: int = 2, n_ctx: int = 512, raw=None,
               head_dim: int = 0, qk_norm: bool = False, biases: bool = False, fused_qkv: bool = False,
               fused_gate_up: bool = False, post_norms: bool = False, extra_meta=()) -> dict:
    """tiny_llama for the llama-family architectures FISH loads (model.cpp:116-118):
    `arch` names the metadata keys ("qwen3" and "qwen2" get NeoX RoPE from FISH);
    head_dim != 0 writes attention.key_length / value_length, so n_head * head_dim
    may differ from n_embd (as in Qwen-3); qk_norm adds the per-head attn_q_norm /
    attn_k_norm vectors (model.cpp:335-341); biases adds attn_q / attn_k / attn_v
    biases (model.cpp:344-346); fused_qkv writes one attn_qkv [q|k|v] tensor and
    fused_gate_up one ffn_up of 2 n_ff rows, gate first, with no ffn_gate (Phi-3,
    model.cpp:253, 1481-1490), both in the q / gate type; post_norms adds Gemma-2's
    post_attention_norm / post_ffw_norm (model.cpp:322-326); extra_meta appends
    (key under the arch, type, value) entries."""
    import imurun_amd as fh

    rng = np.random.default_rng(seed)
    toks, scores, ttypes = spm_vocab()
    vocab = len(toks)
    head_dim = head_dim or n_embd // n_head
    qd = head_dim * n_head
    kv = head_dim * n_head_kv

    def mat(name, t, n_out, n_in, std=0.02):
        w = rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(std)
        if t == fh.F32:
            data = w.tobytes()
        elif t in (fh.Q8_0, fh.Q4_0, fh.Q4_K, fh.Q5_K, fh.Q6_K):
            data = fh.quantize_rows(t, w).tobytes()
        else:
            data = raw(t, n_out, n_in, int(rng.integers(1 << 30))).tobytes()
        return (name, (n_in, n_out), t, data)

    def norm(name, n=n_embd):
        w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        return (name, (n,), fh.F32, w.tobytes())

    def bias(name, n):
        w = (0.1 * rng.standard_normal(n)).astype(np.float32)
        return (name, (n,), fh.F32, w.tobytes())

    tensors = [mat("token_embd.weight", types["embd"], vocab, n_embd, 1.0), norm("output_norm.weight"),
               mat("output.weight", types["output"], vocab, n_embd)]
    for i in range(n_layers):
        p = f"blk.{i}."
        tensors += [
            norm(p + "attn_norm.weight"), norm(p + "ffn_norm.weight"),
        ]
        # (drawn in q, k, v, o, gate, up, down order: the seeded models stay the same)
        if fused_qkv:
            tensors += [mat(p + "attn_qkv.weight", types["q"], qd + 2 * kv, n_embd)]
        else:
            tensors += [mat(p + "attn_q.weight", types["q"], qd, n_embd),
                        mat(p + "attn_k.weight", types["k"], kv, n_embd),
                        mat(p + "attn_v.weight", types["v"], kv, n_embd)]
        tensors += [mat(p + "attn_output.weight", types["o"], n_embd, qd)]
        if fused_gate_up:
            tensors += [mat(p + "ffn_up.weight", types["gate"], 2 * n_ff, n_embd)]
        else:
            tensors += [mat(p + "ffn_gate.weight", types["gate"], n_ff, n_embd),
                        mat(p + "ffn_up.weight", types["up"], n_ff, n_embd)]
        tensors += [mat(p + "ffn_down.weight", types["down"], n_embd, n_ff)]
        if post_norms:
            tensors += [norm(p + "post_attention_norm.weight"), norm(p + "post_ffw_norm.weight")]
        if qk_norm:
            tensors += [norm(p + "attn_q_norm.weight", head_dim), norm(p + "attn_k_norm.weight", head_dim)]
        if biases:
            tensors += [bias(p + "attn_q.bias", qd), bias(p + "attn_k.bias", kv), bias(p + "attn_v.bias", kv)]
    a = arch
    meta = [
        ("general.architecture", STR, arch),
        ("general.alignment", U32, ALIGN),
        (a + ".block_count", U32, n_layers),
        (a + ".embedding_length", U32, n_embd),
        (a + ".feed_forward_length", U32, n_ff),
        (a + ".attention.head_count", U32, n_head),
        (a + ".attention.head_count_kv", U32, n_head_kv),
        (a + ".attention.layer_norm_rms_epsilon", F32, 1e-5),
        (a + ".rope.freq_base", F32, 10000.0),
        (a + ".context_length", U32, n_ctx),
        ("tokenizer.ggml.model", STR, "llama"),
        ("tokenizer.ggml.tokens", ARR, (STR, toks)),
        ("tokenizer.ggml.scores", ARR, (F32, scores)),
        ("tokenizer.ggml.token_type", ARR, (I32, ttypes)),
        ("tokenizer.ggml.bos_token_id", U32, 1),
        ("tokenizer.ggml.eos_token_id", U32, 2),
        ("tokenizer.ggml.unknown_token_id", U32, 0),
    ]
    if head_dim != n_embd // n_head:
        meta += [(a + ".attention.key_length", U32, head_dim), (a + ".attention.value_length", U32, head_dim)]
    meta += [(a + "." + k, kind, v) for k, kind, v in extra_meta]
    write_gguf(path, meta, tensors)
    return {"n_layers": n_layers, "n_embd": n_embd, "n_ff": n_ff, "n_head": n_head, "n_head_kv": n_head_kv,
            "vocab": vocab, "n_ctx": n_ctx, "head_dim": head_dim}
