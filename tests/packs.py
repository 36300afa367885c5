"""Writes Hale expert packs for the tests, in the layout PackWriter produces
(src/expert/pack.rs:1-16, :75-99, :148-190):

  offset 0      b"HALEPACK"
  offset 8      u64 LE length of the JSON header
  offset 16     JSON PackHeader, fields in declaration order, compact
  data_offset   record (MoE layer ordinal o, expert e) at
                data_offset + (o * num_experts + e) * record_stride

data_offset is computed as the writer does: the header is serialised with
data_offset 0 and 32 bytes of slack are added before rounding up to 16 KiB.
"""
import json
import struct

import oracle as O

ALIGN = 16 * 1024
MAGIC = b"HALEPACK"
DTYPE_NAMES = {O.F32: "f32", O.F16: "f16", O.BF16: "bf16", O.Q8_0: "q8_0", O.Q4_0: "q4_0"}


def round_up(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def header_for(dtype: int, hidden: int, inter: int, num_experts: int, moe_layers) -> dict:
    """PackHeader::for_model (src/expert/pack.rs:77-94)."""
    record_bytes = 2 * inter * O.row_bytes(dtype, hidden) + hidden * O.row_bytes(dtype, inter)
    h = {
        "version": 1,
        "dtype": DTYPE_NAMES[dtype],
        "hidden_size": hidden,
        "intermediate_size": inter,
        "num_experts": num_experts,
        "moe_layers": list(moe_layers),
        "record_bytes": record_bytes,
        "record_stride": round_up(record_bytes, ALIGN),
        "data_offset": 0,
    }
    h["data_offset"] = round_up(16 + len(to_json(h)) + 32, ALIGN)
    return h


def to_json(h: dict) -> bytes:
    return json.dumps(h, separators=(",", ":")).encode()


def file_size(h: dict) -> int:
    return h["data_offset"] + len(h["moe_layers"]) * h["num_experts"] * h["record_stride"]


def offset_of(h: dict, layer: int, expert: int) -> int:
    o = h["moe_layers"].index(layer)
    return h["data_offset"] + (o * h["num_experts"] + expert) * h["record_stride"]


def write_pack(path, h: dict, records: dict, header_bytes: bytes | None = None):
    """Creates the file at its full size (zeros where no record is written),
    then writes `records` {(layer, expert): bytes of gate|up|down}."""
    js = to_json(h) if header_bytes is None else header_bytes
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<Q", len(js)))
        f.write(js)
        f.truncate(file_size(h))
        for (layer, expert), rec in records.items():
            assert len(rec) == h["record_bytes"]
            f.seek(offset_of(h, layer, expert))
            f.write(bytes(rec))
