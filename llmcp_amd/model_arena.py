"""The LLMCPWGT arena of a 4B-class Qwen3.5 text model, laid out the way
llmcp-pack lays it out, with synthetic contents.

The reference packer places every tensor with ``WeightLayout::addTensor``
(lib/Model/WeightLayout.cpp:54-87): a 64-byte aligned cursor, and 2-D BF16/F32
tensors whose shape is a packed shape stored as Q8_0 (``q8_0_p4`` bytes,
N * K * 34 / 32) when the arena is quantized.  ``WeightLayout::build``
(:95-265) fixes the order: the tied embedding table, then the layers group
by group (each linear-attention or full-attention layer's norms, mixer
projections, conv and gate parameters, then its MLP), each group padded to
one stride, then the final norm.  The manifest keys are those of
``WeightPacker`` (lib/Model/WeightPacker.cpp:126-160).

The model dimensions are the 4B-class configuration of the reference's
config fixture (tests/unittests/ModelConfigTest.cpp:17-55: hidden 2560,
intermediate 9216, 16 linear key heads and 32 value heads of 128, 16
attention heads and 4 KV heads of 256, vocabulary 248320, three
linear-attention layers per full-attention layer) at 32 layers, which gives
the real model's 426 tensors and 4.47 GB arena (docs/int8-quantization.md:
718-724).  Contents are seeded random bytes: Q8_0 records hold int8 values
in [-127, 127] and f16 scales of N(0, 0.02)-like weights, BF16 and F32
tensors hold small finite values.  This is a model-shaped test and benchmark
input, not a checkpoint.
"""
import json

import numpy as np

HEADER_BYTES = 64
ALIGNMENT = 64

CONFIG_4B = {
    "hidden": 2560, "intermediate": 9216, "vocab": 248320, "layers": 32,
    "full_attention_interval": 4, "linear_key_heads": 16,
    "linear_value_heads": 32, "linear_key_head_dim": 128,
    "linear_value_head_dim": 128, "linear_conv_kernel": 4,
    "attention_heads": 16, "kv_heads": 4, "head_dim": 256,
}


def _align(v):
    return (v + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT


def _packed(shape):
    # isQ8PackedShape (Q8PackedLayout.h:38-42) and the 32-column block rule
    return len(shape) == 2 and shape[0] % 8 == 0 and shape[1] % 32 == 0


def tensor_specs(cfg=CONFIG_4B):
    """(name, shape, source dtype) in WeightLayout::build order, plus the
    number of layer groups."""
    h, f, v = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    qkv = (cfg["linear_key_heads"] * cfg["linear_key_head_dim"] * 2
           + cfg["linear_value_heads"] * cfg["linear_value_head_dim"])
    vdim = cfg["linear_value_heads"] * cfg["linear_value_head_dim"]
    nvh = cfg["linear_value_heads"]
    qout = cfg["attention_heads"] * cfg["head_dim"] * 2
    kv = cfg["kv_heads"] * cfg["head_dim"]
    specs = [("model.language_model.embed_tokens.weight", (v, h), "BF16")]
    interval = cfg["full_attention_interval"]
    groups = cfg["layers"] // interval
    for layer in range(cfg["layers"]):
        p = "model.language_model.layers.%d." % layer
        specs += [(p + "input_layernorm.weight", (h,), "BF16"),
                  (p + "post_attention_layernorm.weight", (h,), "BF16")]
        if layer % interval != interval - 1:  # linear attention
            specs += [(p + "linear_attn.in_proj_qkv.weight", (qkv, h), "BF16"),
                      (p + "linear_attn.in_proj_z.weight", (vdim, h), "BF16"),
                      (p + "linear_attn.in_proj_a.weight", (nvh, h), "BF16"),
                      (p + "linear_attn.in_proj_b.weight", (nvh, h), "BF16"),
                      (p + "linear_attn.conv1d.weight",
                       (qkv, 1, cfg["linear_conv_kernel"]), "BF16"),
                      (p + "linear_attn.dt_bias", (nvh,), "BF16"),
                      (p + "linear_attn.A_log", (nvh,), "F32"),
                      (p + "linear_attn.norm.weight",
                       (cfg["linear_value_head_dim"],), "F32"),
                      (p + "linear_attn.out_proj.weight", (h, vdim), "BF16")]
        else:  # full attention
            specs += [(p + "self_attn.q_proj.weight", (qout, h), "BF16"),
                      (p + "self_attn.k_proj.weight", (kv, h), "BF16"),
                      (p + "self_attn.v_proj.weight", (kv, h), "BF16"),
                      (p + "self_attn.o_proj.weight",
                       (h, cfg["attention_heads"] * cfg["head_dim"]), "BF16"),
                      (p + "self_attn.q_norm.weight", (cfg["head_dim"],), "BF16"),
                      (p + "self_attn.k_norm.weight", (cfg["head_dim"],), "BF16")]
        specs += [(p + "mlp.gate_proj.weight", (f, h), "BF16"),
                  (p + "mlp.up_proj.weight", (f, h), "BF16"),
                  (p + "mlp.down_proj.weight", (h, f), "BF16")]
    specs.append(("model.language_model.norm.weight", (h,), "BF16"))
    return specs, groups


def layout(cfg=CONFIG_4B, quantize=True):
    """Manifest entries (dicts with name, offset, size, dtype, source_size,
    shape), the group stride and the arena size, as WeightLayout::build
    computes them."""
    specs, groups = tensor_specs(cfg)
    per_group = (len(specs) - 2) // groups
    entries = []
    cursor = HEADER_BYTES
    stride = None

    def add(name, shape, dtype):
        nonlocal cursor
        elems = int(np.prod(shape))
        src = elems * (2 if dtype == "BF16" else 4)
        e = {"name": name, "offset": _align(cursor), "size": src,
             "dtype": dtype, "source_size": src, "shape": list(shape)}
        if quantize and _packed(shape):
            e["size"] = shape[0] * shape[1] // 32 * 34
            e["dtype"] = "Q8_0"
        entries.append(e)
        cursor = e["offset"] + e["size"]

    add(*specs[0])
    for g in range(groups):
        start = cursor
        for spec in specs[1 + g * per_group:1 + (g + 1) * per_group]:
            add(*spec)
        nbytes = _align(cursor - start)
        if stride is None:
            stride = nbytes
        assert nbytes == stride, "layer groups differ in size"
        cursor = start + stride
    add(*specs[-1])
    return entries, stride, groups, _align(cursor)


def manifest(entries, stride, groups, total, quantize=True):
    m = {"model": "synthetic-4b", "total_bytes": total,
         "header_bytes": HEADER_BYTES, "group_stride": stride,
         "num_groups": groups, "alignment": ALIGNMENT,
         "quantization": "q8_0" if quantize else "none",
         "tensors": entries}
    if quantize:
        m["block_size"] = 32
        m["quant_layout"] = "q8_0_p4"
    return json.dumps(m).encode() + b"\n"


def synth_q8_records(rng, rows, cols):
    """q8_0_p4 bytes of a [rows, cols] tensor: int8 values in [-127, 127] and
    f16 scales near 0.02 * 2.5 / 127 (the scale of N(0, 0.02) blocks)."""
    groups, blocks = rows // 4, cols // 32
    rec = np.empty((groups * blocks, 136), np.uint8)
    scales = (rng.uniform(0.7, 1.3, (groups * blocks, 4)) * 4.0e-4).astype(np.float16)
    rec[:, :8] = scales.view(np.uint8).reshape(-1, 8)
    rec[:, 8:] = rng.integers(-127, 128, (groups * blocks, 128), dtype=np.int8).view(np.uint8)
    return rec.reshape(-1)


def build_image(cfg=CONFIG_4B, seed=0):
    """The whole file image (header, arena, manifest) as a uint8 array, and
    the manifest entries.  About 4.5 GB at the 32-layer configuration."""
    entries, stride, groups, total = layout(cfg)
    man = manifest(entries, stride, groups, total)
    image = np.zeros(total + len(man), np.uint8)
    rng = np.random.default_rng(seed)
    for e in entries:
        o, n = e["offset"], e["size"]
        if e["dtype"] == "Q8_0":
            image[o:o + n] = synth_q8_records(rng, *e["shape"])
        elif e["dtype"] == "BF16":
            vals = rng.standard_normal(n // 2).astype(np.float32) * 0.1 + 1.0
            image[o:o + n] = (vals.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        else:
            image[o:o + n] = (rng.standard_normal(n // 4).astype(np.float32) * 0.1).view(np.uint8)
    image[total:] = np.frombuffer(man, np.uint8)
    hdr = np.zeros(64, np.uint8)
    hdr[:8] = np.frombuffer(b"LLMCPWGT", np.uint8)
    hdr[8:16] = np.array([1, HEADER_BYTES], np.uint32).view(np.uint8)
    hdr[16:40] = np.array([total, total, len(man)], np.uint64).view(np.uint8)
    image[:64] = hdr
    return image, entries
