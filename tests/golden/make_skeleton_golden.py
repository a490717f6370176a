"""Writes native_skeletons.json: the op skeletons of the native op path and
their SHA-256 fingerprints, computed here in Python (struct + hashlib) from
the reference's published skeleton definitions, independently of the C code.

Header bytes (reference src/ops/include/ops.h:15-30): char[256] nickname
(NUL padded), int32 num_args, int32 arg_dtypes[32] (unused = DATAFLOW_NONE = 0),
little-endian; fingerprint = SHA-256 of those 388 bytes. Nicknames and dtype
lists follow src/set_ops/src/set_native_op_skeletons.c:234-611 and the
strings of src/datatype/src/dataflow_datatype.c:43-78.

Run: python tests/golden/make_skeleton_golden.py
"""
import hashlib
import json
import os
import struct

NAMES = {2: "FP64", 3: "FP32", 4: "FP16", 5: "BF16", 6: "FP8E4M3", 7: "FP8E5M2", 8: "UINT64", 9: "UINT32",
         10: "UINT16", 11: "UINT8", 12: "LONG", 13: "INT", 1: "VOID"}
INT, UINT32, UINT64_S, INT_S, FP32_S, FP32 = 13, 9, 21, 26, 16, 3
F, B = "F", "B"

# op: (nickname form, argument dtypes)
SPECS = {
    "embedding": ("F", [INT_S, INT_S, UINT32, F, F]),
    "rms_norm": ("F", [INT_S, INT_S, FP32_S, F, F, F, FP32, FP32]),
    "rms_norm_bwd_x": ("FB", [INT_S, INT_S, FP32_S, FP32, FP32, F, F, B, B]),
    "rms_norm_bwd_w": ("FB", [INT_S, INT_S, FP32_S, FP32, F, B, B]),
    "rope": ("F", [UINT64_S, INT_S, INT_S, INT_S, INT_S, INT, F, F]),
    "rope_bwd_x": ("B", [UINT64_S, INT_S, INT_S, INT_S, INT_S, INT, B, B]),
    "copy_to_seq_context": ("F", [UINT64_S, INT_S, INT_S, F, F, INT, 8, INT]),
    "swiglu": ("F", [INT_S, INT_S, F, F, F]),
    "swiglu_bwd_x": ("FB", [INT_S, INT_S, F, F, B, B, B]),
    "softmax": ("FB", [INT_S, INT_S, F, B]),
    "cross_entropy_loss": ("B", [INT_S, INT_S, B, UINT32]),
    # the fused ops of this library (no reference counterpart)
    "rms_norm_bwd": ("FB", [INT_S, INT_S, FP32_S, FP32, F, F, B, B, FP32]),
    "softmax_cross_entropy_loss": ("F", [INT_S, INT_S, F, UINT32, FP32, FP32]),
    "rope_copy_to_seq_context": ("F", [UINT64_S, INT_S, INT_S, INT_S, INT_S, INT, F, F, F, 8, INT]),
}

# the reference's register_native_ops variants (set_native_op_skeletons.c:5-184)
FWD5 = [3, 4, 5, 6, 7]
BWD3 = [3, 4, 5]
COMBOS7 = [(3, 3), (4, 4), (5, 5), (6, 4), (6, 5), (7, 4), (7, 5)]
REFERENCE_VARIANTS = ([("embedding", f, 0) for f in FWD5] + [("rms_norm", f, 0) for f in FWD5] +
                      [("rms_norm_bwd_x", f, b) for f, b in COMBOS7] + [("rms_norm_bwd_w", f, b) for f, b in COMBOS7] +
                      [("rope", f, 0) for f in FWD5] + [("rope_bwd_x", 0, b) for b in BWD3] +
                      [("swiglu", f, 0) for f in FWD5] + [("swiglu_bwd_x", f, b) for f, b in COMBOS7] +
                      [("softmax", f, b) for f, b in COMBOS7] + [("cross_entropy_loss", 0, b) for b in BWD3])
FUSED_VARIANTS = ([("rms_norm_bwd", d, d) for d in BWD3] + [("softmax_cross_entropy_loss", d, 0) for d in BWD3] +
                  [("rope_copy_to_seq_context", d, 0) for d in BWD3])


def header(op, fwd, bwd):
    form, args = SPECS[op]
    name = lambda dt: NAMES.get(dt, "UNKNOWN")
    if form == "F":
        nick = "%s_%s" % (op, name(fwd))
    elif form == "B":
        nick = "%s_%s" % (op, name(bwd))
    else:
        nick = "%s_%s_%s" % (op, name(fwd), name(bwd))
    dts = [fwd if a == F else bwd if a == B else a for a in args]
    raw = nick.encode()[:255].ljust(256, b"\0") + struct.pack("<i", len(dts)) + struct.pack("<32i", *(dts + [0] * (32 - len(dts))))
    assert len(raw) == 388
    return nick, raw


def main():
    out = []
    for op, f, b in REFERENCE_VARIANTS + FUSED_VARIANTS:
        nick, raw = header(op, f, b)
        out.append({"op": op, "fwd_dt": f, "bwd_dt": b, "nickname": nick, "sha256": hashlib.sha256(raw).hexdigest(),
                    "in_reference": (op, f, b) in REFERENCE_VARIANTS})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native_skeletons.json")
    with open(path, "w") as fh:
        json.dump({"generator": "tests/golden/make_skeleton_golden.py (struct + hashlib)", "skeletons": out}, fh, indent=1)
    print("wrote %d skeletons to %s" % (len(out), path))


if __name__ == "__main__":
    main()
