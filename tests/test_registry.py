"""Host-side registry: datatype enum and strings, SHA-256 fingerprints, op
skeletons, and the op table. Checked against FIPS 180-4 known answers, the
committed golden digests (tests/golden/native_skeletons.json, built with
hashlib), and — when oracle/_ref was built from /root/reference — the
reference's own host C."""
import ctypes
import hashlib
import json
import os
import random

import numpy as np
import pytest

from support import REF_HOST_LIB, ROOT

from dataflow_lib_amd import api

GOLDEN = os.path.join(ROOT, "tests", "golden", "native_skeletons.json")


def ref_lib():
    if not os.path.exists(REF_HOST_LIB):
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")
    L = ctypes.CDLL(REF_HOST_LIB)
    L.set_native_op_skeleton.argtypes = [ctypes.POINTER(api.OpSkeleton), ctypes.c_char_p, ctypes.c_int, ctypes.c_int]
    L.dataflow_datatype_as_string.restype = ctypes.c_char_p
    L.dataflow_sizeof_element.restype = ctypes.c_size_t
    return L


# ---------------- datatypes ----------------

ENUM_ORDER = ["NONE", "VOID", "FP64", "FP32", "FP16", "BF16", "FP8E4M3", "FP8E5M2", "UINT64", "UINT32", "UINT16",
              "UINT8", "LONG", "INT", "BOOL", "FP64_SCALAR", "FP32_SCALAR", "FP16_SCALAR", "BF16_SCALAR",
              "FP8E4M3_SCALAR", "FP8E5M2_SCALAR", "UINT64_SCALAR", "UINT32_SCALAR", "UINT16_SCALAR", "UINT8_SCALAR",
              "LONG_SCALAR", "INT_SCALAR", "BOOL_SCALAR"]


def test_enum_values_fixed():
    for v, name in enumerate(ENUM_ORDER):
        assert getattr(api, "DATAFLOW_" + name) == v


def test_datatype_strings_and_sizes():
    sizes = {2: 8, 3: 4, 4: 2, 5: 2, 6: 1, 7: 1, 8: 8, 9: 4, 10: 2, 11: 1, 12: 8, 13: 4}
    for dt in range(-1, 30):
        assert api.sizeof_element(dt) == sizes.get(dt, 0)
        exp = {1: "VOID", 12: "LONG", 13: "INT"}.get(dt, ENUM_ORDER[dt] if 2 <= dt <= 11 else "UNKNOWN")
        assert api.datatype_as_string(dt) == exp


def test_datatype_matches_reference_build():
    L = ref_lib()
    for dt in range(-1, 30):
        assert L.dataflow_datatype_as_string(dt).decode() == api.datatype_as_string(dt)
        assert L.dataflow_sizeof_element(dt) == api.sizeof_element(dt)


def test_convert_datatype_roundtrip():
    L = api.lib()
    x = np.random.default_rng(0).standard_normal(10001).astype(np.float32) * 100
    x[:6] = [0.0, -0.0, np.inf, -np.inf, 65504.0, 1e-8]
    h = np.empty(x.size, np.float16)
    assert L.dataflow_convert_datatype(h.ctypes.data, x.ctypes.data, api.DATAFLOW_FP16, api.DATAFLOW_FP32, x.size, 4) == 0
    assert np.array_equal(h.view(np.uint16), x.astype(np.float16).view(np.uint16))
    b = np.empty(x.size, np.uint16)
    assert L.dataflow_convert_datatype(b.ctypes.data, x.ctypes.data, api.DATAFLOW_BF16, api.DATAFLOW_FP32, x.size, 3) == 0
    from support import f32_to_bf16_bits, bf16_bits_to_f32
    assert np.array_equal(b, f32_to_bf16_bits(x))
    back = np.empty(x.size, np.float32)
    assert L.dataflow_convert_datatype(back.ctypes.data, b.ctypes.data, api.DATAFLOW_FP32, api.DATAFLOW_BF16, x.size, 2) == 0
    assert np.array_equal(back.view(np.uint32), bf16_bits_to_f32(b).view(np.uint32))
    assert L.dataflow_convert_datatype(back.ctypes.data, b.ctypes.data, api.DATAFLOW_UINT8, api.DATAFLOW_BF16, 4, 1) == -1


# ---------------- fingerprints ----------------

def digest(data, kind):
    L = api.lib()
    n = L.get_fingerprint_num_bytes(kind)
    out = (ctypes.c_uint8 * 64)()
    buf = ctypes.create_string_buffer(data, len(data))
    L.do_fingerprinting(buf, len(data), out, kind)
    return bytes(out[:n])


@pytest.mark.parametrize("msg,hexd", [
    (b"abc", "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"),
    (b"", "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"),
    (b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
     "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"),
])
def test_sha256_known_answers(msg, hexd):
    assert digest(msg, 0).hex() == hexd


def test_other_digest_kinds_known_answers():
    assert digest(b"abc", 2).hex() == "a9993e364706816aba3e25717850c26c9cd0d89d"
    assert digest(b"abc", 3).hex() == "900150983cd24fb0d6963f7d28e17f72"
    assert digest(b"abc", 1).hex() == hashlib.sha512(b"abc").hexdigest()


def test_least_sig64():
    fp = (ctypes.c_uint8 * 32)(*range(32))
    assert api.lib().fingerprint_to_least_sig64(fp, 32) == int.from_bytes(bytes(range(24, 32)), "big")


def golden():
    with open(GOLDEN) as f:
        return json.load(f)["skeletons"]


def test_skeletons_match_golden_digests():
    g = golden()
    assert len(g) == 63 and sum(s["in_reference"] for s in g) == 54
    for s in g:
        sk = api.native_op_skeleton(s["op"], s["fwd_dt"], s["bwd_dt"])
        assert sk.header.op_nickname.decode() == s["nickname"]
        assert bytes(sk.fingerprint).hex() == s["sha256"]
        assert hashlib.sha256(api.header_bytes(sk)).hexdigest() == s["sha256"]


def test_cached_fingerprints_match_fresh_digests():
    """Fingerprints are cached per (op, fwd, bwd) after the first build; later
    builds return the same bytes, equal to SHA-256 of the rebuilt header."""
    for s in golden():
        for _ in range(3):
            sk = api.native_op_skeleton(s["op"], s["fwd_dt"], s["bwd_dt"])
            assert bytes(sk.fingerprint).hex() == s["sha256"] == hashlib.sha256(api.header_bytes(sk)).hexdigest()
    # a dtype outside the cache's range is still fingerprinted
    sk = api.native_op_skeleton("rope", 40)
    assert bytes(sk.fingerprint) == hashlib.sha256(api.header_bytes(sk)).digest()


def test_skeletons_match_reference_build_all_dtype_pairs():
    L = ref_lib()
    ops = ["embedding", "rms_norm", "rms_norm_bwd_x", "rms_norm_bwd_w", "rope", "rope_bwd_x", "copy_to_seq_context",
           "swiglu", "swiglu_bwd_x", "softmax", "cross_entropy_loss"]
    for op in ops:
        for f in range(0, 28):
            for b in (0, 3, 4, 5, 6, 7, 13):
                mine = api.native_op_skeleton(op, f, b)
                ref = api.OpSkeleton()
                assert L.set_native_op_skeleton(ctypes.byref(ref), op.encode(), f, b) == 0
                assert bytes(mine) == bytes(ref), (op, f, b)


def test_unknown_op_skeleton():
    with pytest.raises(ValueError):
        api.native_op_skeleton("matmul", api.DATAFLOW_BF16)


def test_header_layout():
    assert ctypes.sizeof(api.OpSkeletonHeader) == 388
    assert ctypes.sizeof(api.OpSkeleton) == 420
    assert ctypes.sizeof(api.Op) == 420 + 4 + 32 * 8


# ---------------- op table ----------------

def make_table(L, size_min=8, size_max=64, key_bytes=8, val_bytes=8, load=0.75, shrink=0.25, hash_fn=None):
    L.init_table.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                             ctypes.c_uint64, ctypes.c_float, ctypes.c_float]
    L.insert_table.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    L.find_table.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_bool, ctypes.c_void_p]
    L.find_table.restype = ctypes.c_long
    L.remove_table.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    L.destroy_table.argtypes = [ctypes.c_void_p]
    t = api.Table()
    assert L.init_table(ctypes.byref(t), ctypes.cast(hash_fn, ctypes.c_void_p), key_bytes, val_bytes,
                        size_min, size_max, load, shrink) == 0
    return t


# a deliberately clustering hash: key mod 4 scaled, so probe chains wrap and collide
_clustered = api.HashFunc(lambda key, size: (ctypes.cast(key, ctypes.POINTER(ctypes.c_uint64))[0] % 4) * (size // 4 + 1) % size)


def run_ops(L, seed, n_ops=3000, hash_fn=_clustered, **kw):
    t = make_table(L, hash_fn=hash_fn, **kw)
    rnd = random.Random(seed)
    model, trace = {}, []
    for _ in range(n_ops):
        k = rnd.randrange(1, 80)
        key = ctypes.c_uint64(k)
        op = rnd.random()
        if op < 0.5:
            v = ctypes.c_uint64(rnd.randrange(1 << 40))
            rc = L.insert_table(ctypes.byref(t), ctypes.byref(key), ctypes.byref(v))
            if rc == 0:
                model[k] = v.value
            trace.append(("ins", k, rc))
        elif op < 0.8:
            out = ctypes.c_uint64(0)
            idx = L.find_table(ctypes.byref(t), ctypes.byref(key), True, ctypes.byref(out))
            assert (idx != -1) == (k in model)
            if idx != -1:
                assert out.value == model[k]
            trace.append(("find", k, idx))
        else:
            out = ctypes.c_uint64(0)
            rc = L.remove_table(ctypes.byref(t), ctypes.byref(key), ctypes.byref(out))
            assert (rc == 0) == (k in model)
            if rc == 0:
                assert out.value == model.pop(k)
            trace.append(("rm", k, rc))
        assert t.cnt == len(model)
    L.destroy_table(ctypes.byref(t))
    return trace


def test_table_against_dict_model():
    for seed in range(5):
        run_ops(api.lib(), seed)


def test_table_duplicate_and_full():
    L = api.lib()
    t = make_table(L, size_min=4, size_max=4, load=1.0, shrink=0.0, hash_fn=_clustered)
    for k in range(1, 5):
        assert L.insert_table(ctypes.byref(t), ctypes.byref(ctypes.c_uint64(k)), ctypes.byref(ctypes.c_uint64(k))) == 0
    assert L.insert_table(ctypes.byref(t), ctypes.byref(ctypes.c_uint64(9)), ctypes.byref(ctypes.c_uint64(9))) == -1
    assert L.insert_table(ctypes.byref(t), ctypes.byref(ctypes.c_uint64(2)), ctypes.byref(ctypes.c_uint64(2))) == -1
    for k in range(1, 5):
        assert L.find_table(ctypes.byref(t), ctypes.byref(ctypes.c_uint64(k)), False, None) != -1
    L.destroy_table(ctypes.byref(t))


def test_table_slot_indices_match_reference_build():
    """same insert policy (first empty slot from the hash, wrapping), same
    backward-shift removal, same growth and shrink: identical return codes and
    slot indices for every operation. The table never fills up here: at
    cnt == size == max_size the reference's find_table probes only up to the
    end of the array without wrapping (table.c:419-433) and misses keys whose
    chain wrapped, which the dict-model test above covers for this library."""
    L = ref_lib()
    for seed in range(4):
        mine = run_ops(api.lib(), 100 + seed, size_max=512)
        theirs = run_ops(L, 100 + seed, size_max=512)
        assert mine == theirs


def test_external_matmul_skeleton_matches_reference_build():
    """the matmul skeleton (19 args) is byte-identical to the reference's, so
    an Op built by either side resolves to the same table entry"""
    L = ref_lib()
    L.set_external_matmul_skeleton.argtypes = [ctypes.POINTER(api.OpSkeleton)]
    api.lib().set_external_matmul_skeleton.argtypes = [ctypes.POINTER(api.OpSkeleton)]
    mine, ref = api.OpSkeleton(), api.OpSkeleton()
    api.lib().set_external_matmul_skeleton(ctypes.byref(mine))
    L.set_external_matmul_skeleton(ctypes.byref(ref))
    assert bytes(mine) == bytes(ref)
    assert mine.header.op_nickname.decode() == "matmul" and mine.header.num_args == 19
    digest = hashlib.sha256(bytes(mine.header)).digest()
    assert bytes(mine.fingerprint)[:32] == digest
