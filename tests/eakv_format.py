"""The .eakv file format restated independently of both writers under test
(eakv_amd/csrc/io.c and oracle/eakv_oracle.c), from the reference's packed
header struct and its save/load code (src/io.c:6-160).

Header, 512 bytes, `#pragma pack(push, 1)` little endian (io.c:11-28):
  char magic[4]; u16 version; u16 quant_scheme; u32 group_size;
  u16 orig_dtype; u32 n_layers; u32 n_heads; u32 head_dim; u32 seq_len;
  u32 max_seq_len; i16 compression; char model_hash[32];
  char tokenizer_hash[32]; u64 checksum
then zeros to 512 (io.c:49-50).  save writes version 1, quant 0, group 64,
dtype 0, max_seq_len = seq_len (io.c:54-66), then n_layers*2 u64 block
offsets (io.c:70-80), zeros to the 64-byte aligned data start (:82-84), and
per (layer, kv) a block weights|scales|biases of n_groups =
n_heads*head_dim*seq_len/64 groups, zero padded to 64 bytes (:86-98).  load
checks magic and version (io.c:115-121) and reads each block at its table
offset (:133-144).
"""
import struct

HEADER = struct.Struct("<4sHHIHIIIIIh32s32sQ")
HEADER_SIZE = 512
FIELDS = ("magic", "version", "quant_scheme", "group_size", "orig_dtype", "n_layers",
          "n_heads", "head_dim", "seq_len", "max_seq_len", "compression", "model_hash",
          "tokenizer_hash", "checksum")


def align64(x):
    return (x + 63) & ~63


def parse(data: bytes):
    """(header dict, list of block offsets, n_groups) of a file's bytes."""
    h = dict(zip(FIELDS, HEADER.unpack_from(data, 0)))
    n = h["n_layers"] * 2
    offs = list(struct.unpack_from(f"<{n}Q", data, HEADER_SIZE))
    n_groups = h["n_heads"] * h["head_dim"] * h["seq_len"] // 64
    return h, offs, n_groups


def block(data: bytes, off: int, n_groups: int):
    """weights (bytes), scales and biases (bytes) of the block at off."""
    w = data[off:off + 32 * n_groups]
    s = data[off + 32 * n_groups:off + 36 * n_groups]
    b = data[off + 36 * n_groups:off + 40 * n_groups]
    return w, s, b


def build(n_layers, n_heads, head_dim, seq_len, blocks, order=None, gap=0, magic=b"EAKV",
          version=1):
    """File bytes for `blocks[l*2+kv]` = (weights, scales, biases) bytes, each
    n_groups groups in [head][pos][group] order.  Blocks are written in
    `order` (default: table order) with `gap` extra bytes between them (the
    table says where each one is)."""
    hdr = bytearray(HEADER_SIZE)
    HEADER.pack_into(hdr, 0, magic, version, 0, 64, 0, n_layers, n_heads, head_dim, seq_len,
                     seq_len, 0, bytes(32), bytes(32), 0)
    n = n_layers * 2
    start = align64(HEADER_SIZE + 8 * n)
    order = list(range(n)) if order is None else list(order)
    offs = [0] * n
    body = bytearray()
    for i in order:
        w, s, b = blocks[i]
        offs[i] = start + len(body)
        raw = bytes(w) + bytes(s) + bytes(b)
        body += raw + bytes(align64(len(raw)) - len(raw) + gap)
    table = struct.pack(f"<{n}Q", *offs)
    return bytes(hdr) + table + bytes(start - HEADER_SIZE - len(table)) + bytes(body)
