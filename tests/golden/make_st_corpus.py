"""Writes tests/golden/st_corpus/: small safetensors files for the reader's
robustness tests (tests/test_st_corpus.py, also run under the sanitizers).

Layout (SafeTensors.swift:41-118, 217-240): little-endian u64 header length,
a JSON object header, then the data.  Hand-made cases cover each field the
reader checks; the mutated cases are a valid file truncated at many lengths
and with seeded byte flips and byte overwrites in its header.  expect.json
maps each file to "ok" (opens; every tensor reads back) or to a fragment of
the error message.

    python tests/golden/make_st_corpus.py
"""
import json
import os
import random
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "st_corpus")


def st(header_obj=None, data=b"", raw_header=None, hlen=None, pad=True):
    h = raw_header if raw_header is not None else json.dumps(header_obj).encode()
    if pad and raw_header is None:
        h += b" " * ((8 - len(h) % 8) % 8)
    n = len(h) if hlen is None else hlen
    return struct.pack("<Q", n) + h + data


def t(dtype, shape, a, b):
    return {"dtype": dtype, "shape": shape, "data_offsets": [a, b]}


def main():
    os.makedirs(OUT, exist_ok=True)
    for f in os.listdir(OUT):
        os.remove(os.path.join(OUT, f))
    data = bytes(range(48))
    good = st({"a": t("F32", [2, 3], 0, 24), "b": t("U8", [24], 24, 48),
               "__metadata__": {"format": "mlx"}}, data)
    cases = {
        # hand-made: (bytes, expected)
        "good": (good, "ok"),
        "empty_file": (b"", "too short"),
        "seven_bytes": (b"\x08\x00\x00\x00\x00\x00\x00", "too short"),
        "hlen_zero": (st(raw_header=b"", hlen=0), "not a JSON object"),
        "hlen_past_end": (st({"a": t("U8", [1], 0, 1)}, b"\x00", hlen=4096), "header length"),
        "hlen_huge": (st({"a": t("U8", [1], 0, 1)}, b"\x00", hlen=2 ** 63 + 5), "header length"),
        "no_tensors": (st({}), "ok"),
        "only_metadata": (st({"__metadata__": {"k": "v"}}), "ok"),
        "json_array": (st(raw_header=b"[1, 2, 3]"), "not a JSON object"),
        "json_null": (st(raw_header=b"null    "), "not a JSON object"),
        "json_unterminated": (st(raw_header=b'{"a": {"dtype": "F32"'), "not a JSON object"),
        "json_deep": (st(raw_header=b'{"a":' + b"[" * 5000 + b"]" * 5000 + b"}"),
                      "not a JSON object"),
        "json_bad_escape": (st(raw_header=b'{"a\\q": 1}'), "not a JSON object"),
        "json_trailing": (st(raw_header=b'{"x": 1} }'), "not a JSON object"),
        # entries that are not tensor objects are skipped, as the reference's
        # `guard ... else { continue }` does (SafeTensors.swift:58-63)
        "missing_dtype": (st({"a": {"shape": [1], "data_offsets": [0, 1]}}, b"\x00"), "ok"),
        "missing_offsets": (st({"a": {"dtype": "U8", "shape": [1]}}, b"\x00"), "ok"),
        "shape_not_list": (st({"a": {"dtype": "U8", "shape": "1", "data_offsets": [0, 1]}},
                              b"\x00"), "ok"),
        "shape_float": (st({"a": t("U8", [1.5], 0, 1)}, b"\x00"), "bad shape"),
        "shape_negative": (st({"a": t("U8", [-1], 0, 0)}), "bad shape"),
        "shape_overflow": (st({"a": t("F32", [2 ** 40, 2 ** 40], 0, 4)}, b"\x00" * 4),
                           "do not match"),
        "shape_nine_dims": (st({"a": t("U8", [1] * 9, 0, 1)}, b"\x00"), "more than 8"),
        "offsets_reversed": (st({"a": t("U8", [0], 4, 0)}, b"\x00" * 4), "outside the file"),
        "offsets_past_end": (st({"a": t("U8", [8], 0, 8)}, b"\x00" * 4), "outside the file"),
        "offsets_huge": (st({"a": t("U8", [1], 2 ** 64 - 1, 2 ** 64)}, b"\x00"),
                         "outside the file"),
        "size_mismatch": (st({"a": t("F32", [3], 0, 8)}, b"\x00" * 8), "do not match"),
        "duplicate_name": (st(raw_header=b'{"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]},'
                                         b'"a":{"dtype":"U8","shape":[1],"data_offsets":[1,2]}}  ',
                              data=b"\x00\x01"), "duplicate tensor name"),
        "unknown_dtype": (st({"a": t("F64", [1], 0, 8), "b": t("U8", [1], 8, 9)}, b"\x00" * 9),
                          "ok"),
        "empty_name": (st({"": t("U8", [1], 0, 1)}, b"\x07"), "ok"),
        "zero_size_tensor": (st({"a": t("F16", [0, 5], 0, 0)}), "ok"),
    }
    # truncations of the good file at every 5th length
    for n in range(0, len(good), 5):
        cases[f"trunc_{n:03d}"] = (good[:n], None)
    # seeded mutations of the header bytes
    rng = random.Random(20261202)
    hl = struct.unpack("<Q", good[:8])[0]
    for i in range(40):
        b = bytearray(good)
        for _ in range(rng.randint(1, 4)):
            j = rng.randrange(8, 8 + hl)
            if rng.random() < 0.5:
                b[j] ^= 1 << rng.randrange(8)
            else:
                b[j] = rng.choice(b'{}[]":,0123456789-e.tfn \\')
        cases[f"mut_{i:02d}"] = (bytes(b), None)
    expect = {}
    for name, (raw, exp) in cases.items():
        with open(os.path.join(OUT, name + ".safetensors"), "wb") as f:
            f.write(raw)
        expect[name] = exp
    with open(os.path.join(OUT, "expect.json"), "w") as f:
        json.dump(expect, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
