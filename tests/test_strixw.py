"""strixw (the converted-weights file): the oracle's parser and hash, and the library's C++ reader / writer, against
the fixture and hash vectors the REFERENCE's own formats/strixw.cpp wrote (tests/golden/make_strixw.py). Host code
only: nothing here touches a GPU."""
import os

import numpy as np
import pytest

import oracle.strixw as ostrixw
from strixite_amd import StrixError
from strixite_amd import strixw

GOLD = os.path.join(os.path.dirname(__file__), "golden")
FIXTURE = os.path.join(GOLD, "layers.strixw")


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLD, "strixw.npz"))


def test_hash_matches_reference(orc, gold):
    blob = gold["hash_blob"]
    for n, want in zip(gold["hash_lengths"], gold["hash_values"]):
        b = blob[:n]
        assert ostrixw.hash64(b) == int(want), n
        assert strixw.hash64(b) == int(want), n
    # the reference's streaming hasher over any split equals its one-shot hash (strixite formats/strixw.cpp:240-246)
    whole = gold["hash_values"][list(gold["hash_lengths"]).index(1000)]
    assert np.all(gold["piece_values"] == whole)


def test_hash_sensitivity(orc):
    """A flipped bit in any position, or one more zero byte, changes the hash (the length seeds the lanes)."""
    rng = np.random.default_rng(3)
    b = rng.integers(0, 256, 77, dtype=np.uint8)
    h = strixw.hash64(b)
    for i in (0, 31, 32, 63, 64, 72, 76):
        c = b.copy()
        c[i] ^= 1
        assert strixw.hash64(c) != h
    assert strixw.hash64(np.concatenate([b, [0]]).astype(np.uint8)) != h


def listing(tensors):
    return [(t.name, t.encoding, list(t.shape), t.group_size, t.experts, [tuple(p) for p in t.parts],
             [tuple(c) for c in t.components]) for t in tensors]


def oracle_listing(f):
    return [(t["name"], ostrixw.ENCODINGS[t["encoding"]], t["shape"], t["group_size"], t["experts"], t["parts"],
             t["components"]) for t in f.tensors]


def test_reader_matches_oracle_parser():
    f, o = strixw.StrixwFile(FIXTURE), ostrixw.File(FIXTURE)
    assert listing(f.tensors) == oracle_listing(o)
    assert f.meta == o.meta and f.meta["arch"] == "qwen4exp"
    assert f.version == 4 and f.data_offset == o.data_offset and f.file_bytes == os.path.getsize(FIXTURE)
    f.verify_hashes(3)
    o.verify()
    for t in f.tensors:  # 4096-aligned tensors, 256-aligned components, in index order without overlap
        assert t.components[0][1] % 4096 == 0
        assert all(c[1] % 256 == 0 for c in t.components)
    offs = [(c[1], c[1] + c[2]) for t in f.tensors for c in t.components]
    assert all(a[1] <= b[0] for a, b in zip(offs, offs[1:]))
    g = f.by_name["model.language_model.layers.0.mlp.experts_gate_up"]
    assert g.parts[0][2] == 4 * 256 and g.parts[-1] == ("model.language_model.layers.0.mlp.shared_expert.up_proj.weight",
                                                         4 * 256 + 128, 128)


def test_fixture_holds_the_generator_weights(orc):
    """The oracle parser's layer weights are the seeded generator's (the fixture's source data), component by
    component: q, scale and min in the right order and place."""
    o = ostrixw.File(FIXTURE)
    w = o.moe_layer("model.language_model.layers.0.", 2)
    q, s, m = orc.gen_q(4, orc.tensor_key(7, "gu_q"), orc.tensor_key(7, "gu_s"), 5 * 256, 128, 128)
    assert w["shared_stacked"] and w["E"] == 4 and w["I"] == 128
    assert np.array_equal(w["gu"][1], q) and np.array_equal(w["gu"][2], s) and np.array_equal(w["gu"][3], m)
    w1 = o.moe_layer("model.language_model.layers.1.", 2)
    q, s, m = orc.gen_q(8, orc.tensor_key(8, "sh_dn_q"), orc.tensor_key(8, "sh_dn_s"), 128, 64, 64)
    assert np.array_equal(w1["sh_dn"][1], q) and np.array_equal(w1["sh_dn"][3], m) and w1["I"] == 64


def test_writer_reproduces_reference_file(tmp_path):
    """The library's writer, given the fixture's plan and bytes, writes the reference writer's file byte for byte."""
    o = ostrixw.File(FIXTURE)
    plan = []
    for t in o.tensors:
        plan.append({"name": t["name"], "encoding": ostrixw.ENCODINGS[t["encoding"]], "shape": t["shape"],
                     "group_size": t["group_size"], "experts": t["experts"],
                     "parts": [(s, r) for s, _, r in t["parts"]],
                     "data": {r: o.data(t["name"], r) for r, _, _, _ in t["components"]}})
    out = str(tmp_path / "copy.strixw")
    strixw.write(out, o.meta, plan)
    assert open(out, "rb").read() == o.buf


@pytest.fixture(scope="module")
def corrupt_cases(gold, tmp_path_factory):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_strixw", os.path.join(GOLD, "make_strixw.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    buf = open(FIXTURE, "rb").read()
    d = tmp_path_factory.mktemp("corrupt")
    out = []
    for (name, b), gname, ok_open, ok_verify in zip(mk.corruptions(buf), gold["corrupt_names"],
                                                    gold["corrupt_open_ok"], gold["corrupt_verify_ok"]):
        assert name == gname
        p = str(d / (name + ".strixw"))
        open(p, "wb").write(b)
        out.append((name, p, bool(ok_open), bool(ok_verify)))
    return out


def test_corruptions_as_the_reference_reader(corrupt_cases):
    """Header / index damage, truncation, appended bytes and unreadable versions are refused at open; a flipped
    data byte is refused by the hash check; padding is not hashed - each verdict the reference reader's."""
    for name, p, ok_open, ok_verify in corrupt_cases:
        try:
            f = strixw.StrixwFile(p)
            opened = True
        except StrixError:
            opened = False
        assert opened == ok_open, name
        if opened:
            try:
                f.verify_hashes(2)
                verified = True
            except StrixError as e:
                verified = False
                assert "fails its stored hash" in str(e), name
            assert verified == ok_verify, name
        try:
            o = ostrixw.File(p)
            o_open = True
        except (ValueError, KeyError):
            o_open = False
        if name != "version_0" and name != "version_5":  # the oracle parser does not check the version range
            assert o_open == ok_open, name


def test_writer_refusals(tmp_path):
    base = {"name": "a", "encoding": "q4", "shape": [4, 64], "group_size": 32,
            "data": {"q": np.zeros(128, np.uint8), "scale": np.zeros(8, np.uint16), "min": np.zeros(8, np.uint16)}}
    p = str(tmp_path / "x.strixw")
    strixw.write(p, {}, [base])
    f = strixw.StrixwFile(p)
    assert [c[2] for c in f.tensors[0].components] == [128, 16, 16]
    with pytest.raises(StrixError, match="group size"):
        strixw.write(p, {}, [dict(base, group_size=16)])
    with pytest.raises(StrixError, match="bytes"):
        strixw.write(p, {}, [dict(base, data=dict(base["data"], q=np.zeros(127, np.uint8)))])
    with pytest.raises(StrixError, match="has no data yet"):
        strixw.write(p, {}, [dict(base, data={"q": base["data"]["q"]})])
    with pytest.raises(StrixError, match="more than once"):
        strixw.write(p, {}, [base, base])
    with pytest.raises(StrixError, match="parts"):
        strixw.write(p, {}, [dict(base, parts=[("src", 3)])])


def test_find_absent_tensor():
    import ctypes as C

    from strixite_amd import _lib as L

    h = C.c_void_p()
    L.check(L.lib().strix_strixw_open(FIXTURE.encode(), C.byref(h)))
    try:
        idx = C.c_int64()
        L.check(L.lib().strix_strixw_find(h, b"nope", C.byref(idx)))
        assert idx.value == -1
        L.check(L.lib().strix_strixw_find(h, b"extra.q6", C.byref(idx)))
        assert idx.value == 11  # index order: 3 + 5 MoE tensors, norm, positions, q4cm, q6
    finally:
        L.lib().strix_strixw_close(h)
