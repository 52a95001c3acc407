"""The real-weights path without a GPU: the POISDv1 reader and the host-side weight preparation of
libvgemm.so (include/vgemm_model.h, vela_amd/model.py) against the arrays the fixture's writer put in
tests/golden/tiny_model.poisd and against the oracle's restatement (oracle/model.py) of
src/poisd.cpp:11-54 and src/engine.cu:11-101; the oracle's merges are pinned by the GEMM identities
they exist for."""
import numpy as np
import pytest

import oracle
from oracle import model as om
from tests import refmath as rm
from tests.golden import make_poisd as mp
from vela_amd._lib import VgemmError
from vela_amd.model import DevModel, Poisd

FIXTURE = mp.PATH
BLOCK = mp.BLOCK


def written():
    """{name: array} as the writer produced them (the first of duplicate names)."""
    out = {}
    for n, arr in mp.tensors():
        out.setdefault(n, arr)
    return out


@pytest.fixture(scope="module")
def model():
    m = Poisd()
    m.load(FIXTURE)
    yield m
    m.close()


@pytest.fixture(scope="module")
def ref():
    return om.parse_poisd(FIXTURE.read_bytes())


def test_fixture_is_the_writers_output():
    assert FIXTURE.read_bytes() == mp.encode(mp.tensors()), "tests/golden/tiny_model.poisd is stale: rerun make_poisd"


def test_oracle_parser_against_writer(ref):
    w = written()
    assert set(ref) == set(w)
    for n, arr in w.items():
        dt, dims, got = ref[n]
        assert dt == mp.CODES[arr.dtype] and dims == list(arr.shape), n
        np.testing.assert_array_equal(got, arr, err_msg=n)


def test_library_reader_against_writer(model):
    w = written()
    assert model.names() == sorted(w, key=lambda s: s.encode())
    for n, arr in w.items():
        t = model.get(n)
        assert t.dtype == mp.CODES[arr.dtype] and t.dims == list(arr.shape) and t.count == arr.size, n
        assert t.bytes() == arr.nbytes
        np.testing.assert_array_equal(model.array(n), arr, err_msg=n)
    assert model.blob("tok.vocab") == b"hello\nworld\n"
    assert model.i32s("c.cin") == -77
    np.testing.assert_array_equal(model.i32v("lut.phi"), mp.phi_table().astype(np.int64))
    with pytest.raises(VgemmError, match="missing tensor no.such"):
        model.get("no.such")
    with pytest.raises(VgemmError, match="lut.phi is not int8"):
        model.i8("lut.phi")


def _both(tmp_path, data: bytes, name="f.poisd"):
    """The library's and the oracle's verdicts on the same bytes (message, or None if accepted)."""
    p = tmp_path / name
    p.write_bytes(data)
    m = Poisd()
    try:
        m.load(p)
        lib_msg = None
    except VgemmError as e:
        lib_msg = str(e).split(": ", 1)[1]
    finally:
        m.close()
    try:
        om.parse_poisd(data)
        orc_msg = None
    except om.FormatError as e:
        orc_msg = str(e)
    return lib_msg, orc_msg


def test_reader_errors(tmp_path):
    good = mp.encode(mp.tensors())
    cases = {
        "empty": (b"", "bad magic (not a POISDv1 file)"),
        "short": (good[:11], "bad magic (not a POISDv1 file)"),
        "magic": (b"POISDv2\x00" + good[8:], "bad magic (not a POISDv1 file)"),
        "count only": (good[:12], "truncated model file"),
        "trailing": (good + b"\x00", "trailing data"),
        "count too small": (mp.encode(mp.tensors(), count=len(mp.tensors()) - 1), "trailing data"),
        "count too large": (mp.encode(mp.tensors(), count=len(mp.tensors()) + 1), "truncated model file"),
    }
    # cuts inside the name length, the name, the header, the dims and the data of the first entry
    for cut in (13, 14, 20, 27, 30, 35, 100, len(good) - 1):
        cases[f"cut {cut}"] = (good[:cut], "truncated model file")
    bad_dt = bytearray(mp.encode([("x", np.zeros(3, np.int8))] + mp.tensors()))
    bad_dt[12 + 2 + 1] = 4   # dtype byte of the first entry
    cases["dtype"] = (bytes(bad_dt), "bad dtype")
    cases["required"] = (mp.encode([t for t in mp.tensors() if t[0] != "lut.phi"]), "missing tensor lut.phi")
    for name, (data, want) in cases.items():
        lib_msg, orc_msg = _both(tmp_path, data)
        assert lib_msg == want, f"{name}: library says {lib_msg!r}"
        assert orc_msg == want, f"{name}: oracle says {orc_msg!r}"
    m = Poisd()
    with pytest.raises(VgemmError, match="cannot open .*nope.poisd"):
        m.load(tmp_path / "nope.poisd")


def test_duplicate_names_keep_the_first(tmp_path):
    items = [("dup", np.array([1, 2], np.int32))] + mp.tensors() + [("dup", np.array([9], np.int32))]
    p = tmp_path / "dup.poisd"
    p.write_bytes(mp.encode(items))
    m = Poisd()
    m.load(p)
    np.testing.assert_array_equal(m.i32v("dup"), [1, 2])
    assert list(om.parse_poisd(p.read_bytes())["dup"][2]) == [1, 2]
    m.close()


def test_prepare_matches_oracle(model, ref):
    dm = DevModel()
    dm.prepare(model)
    lins, norms = om.dev_model(ref)
    assert set(dm.lin_names()) == set(lins)
    for name, (W, cst, N, K, conv3) in lins.items():
        L = dm.lin(name)
        assert (L.N, L.K, L.conv3) == (N, K, conv3), name
        assert (L.Np, L.Kp) == W.shape, name
        np.testing.assert_array_equal(L.w_host, W, err_msg=name)
        np.testing.assert_array_equal(L.cst_host, cst, err_msg=name)
        assert L.w == 0 and L.cst == 0   # nothing on a device yet
    for name, (g, beta, den) in norms.items():
        n = dm.norm(name)
        assert n.C == g.size and n.den == den
        np.testing.assert_array_equal(n.g_host, g)
        np.testing.assert_array_equal(n.beta_host, beta)
    assert set(norms) == {mp.RESNET + ".norm1"}
    with pytest.raises(VgemmError, match="no linear te.tok"):
        dm.lin("te.tok")
    with pytest.raises(VgemmError, match="no norm nothing"):
        dm.norm("nothing")


def test_preparation_kinds(model):
    """Which tensors become linears, the padding grid and the 3x3 permutation, against the file."""
    dm = DevModel()
    dm.prepare(model)
    names = set(dm.lin_names())
    assert {"unet.rank3", "unet.no_requant", "te.tok"}.isdisjoint(names)
    assert {BLOCK + ".attn1.to_qkv", BLOCK + ".ff.net.0.proj.ag", BLOCK + ".ff.net.0.proj.agi"} <= names
    L = dm.lin("unet.time_embedding.linear_1")
    assert (L.N, L.K, L.Np, L.Kp, L.conv3) == (70, 40, 128, 48, False)
    w = model.i8("unet.time_embedding.linear_1.w")
    np.testing.assert_array_equal(L.w_host[:70, :40], w)
    assert not L.w_host[70:].any() and not L.w_host[:, 40:].any()
    assert (L.cst_host[70:] == [1, 0, 0, 0]).all()
    np.testing.assert_array_equal(L.cst_host[:70, 3], w.astype(np.int64).sum(1))
    for base, C in ((mp.RESNET + ".conv1", 64), ("unet.conv_in", 8), ("unet.conv_out", 64)):
        L = dm.lin(base)
        assert L.conv3, base
        w = model.i8(base + ".w")
        want = rm.tapmajor_weights(w.reshape(L.N, C, 3, 3))   # [N, C, 3, 3] -> K index (3ky + kx) C + c
        np.testing.assert_array_equal(L.w_host[:L.N, :L.K], want, err_msg=base)
    assert not dm.lin(mp.RESNET + ".conv_shortcut").conv3


def _requant_rows(q, W, cst):
    return rm.requant(rm.dot_rows(q, W), cst, None)


def test_merge_identities(ref):
    """The oracle's merged operands do what the merges are for: a merged QKV product is the three
    products side by side; a GEGLU over the alternating a/g rows is the GEGLU formula applied to
    separate a and g products."""
    lins, _ = om.dev_model(ref)
    r = np.random.default_rng(5)
    q = r.integers(-32767, 32768, (6, 64)).astype(np.int16)
    parts = [lins[f"{BLOCK}.attn1.{p}"] for p in ("to_q", "to_k", "to_v")]
    Wm, cm, N, K, _ = lins[f"{BLOCK}.attn1.to_qkv"]
    got = oracle.gemm(oracle.SRC_I16, Mreal=6, Nreal=N, Kp=Wm.shape[1], w=Wm, cst=cm, q16=q)
    want = np.concatenate([_requant_rows(q, P[0][:P[2], :K], P[1][:P[2]]) for P in parts], axis=1)
    np.testing.assert_array_equal(got, want.astype(np.int64))
    for P, lo in zip(parts, (0, 64, 128)):   # and [q; k; v] stacked is what "ag" does too
        np.testing.assert_array_equal(Wm[lo:lo + 64], P[0][:64])
    L = ref["lut.phi"][2].astype(np.int32)
    a_, g_ = lins[f"{BLOCK}.ff.net.0.proj.a"], lins[f"{BLOCK}.ff.net.0.proj.g"]
    Wi, ci, Ni, _, _ = lins[f"{BLOCK}.ff.net.0.proj.agi"]
    got = oracle.gemm(oracle.SRC_I16, Mreal=6, Nreal=Ni, Kp=Wi.shape[1], w=Wi, cst=ci, q16=q, epi=oracle.EPI_GEGLU, Lphi=L)
    ya, yg = _requant_rows(q, a_[0][:96, :64], a_[1][:96]), _requant_rows(q, g_[0][:96, :64], g_[1][:96])
    want = np.array([[rm.geglu(ya[i, c], yg[i, c], L) for c in range(96)] for i in range(6)], dtype=np.int64)
    np.testing.assert_array_equal(got, want)
    Wag = lins[f"{BLOCK}.ff.net.0.proj.ag"][0]
    np.testing.assert_array_equal(Wag[:96], a_[0][:96])
    np.testing.assert_array_equal(Wag[96:192], g_[0][:96])


def test_merge_errors():
    lin = lambda N, K: (np.zeros(((N + 63) // 64 * 64, (K + 15) // 16 * 16), np.int8), np.zeros(((N + 63) // 64 * 64, 4), np.int32), N, K, False)
    with pytest.raises(om.FormatError, match="mergeLins: K mismatch"):
        om.merge_lins({"a": lin(8, 16), "b": lin(8, 32)}, ["a", "b"], False)
    with pytest.raises(om.FormatError, match="mergeLins interleave: N mismatch"):
        om.merge_lins({"a": lin(8, 16), "b": lin(9, 16)}, ["a", "b"], True)
    assert om.merge_lins({"a": lin(8, 16)}, ["a", "b"], False) is None


def test_library_merge_errors(tmp_path):
    items = mp.tensors()
    # to_k with a different K: the reference throws "mergeLins: K mismatch" from DevModel::load
    items = [(n, (a[:, :32].copy() if n == f"{BLOCK}.attn1.to_k.w" else a)) for n, a in items]
    p = tmp_path / "kmis.poisd"
    p.write_bytes(mp.encode(items))
    m = Poisd()
    m.load(p)
    with pytest.raises(VgemmError, match="mergeLins: K mismatch"):
        DevModel().prepare(m)
    m.close()
    # a 3x3 convolution whose K is not 9C (src/engine.cu:31)
    items = mp.tensors()
    items = [(n, (a[:, :10].copy() if n == mp.RESNET + ".conv2.w" else a)) for n, a in items]
    p = tmp_path / "k9.poisd"
    p.write_bytes(mp.encode(items))
    m = Poisd()
    m.load(p)
    with pytest.raises(VgemmError, match="conv weight K not multiple of 9: unet.down_blocks.0.resnets.0.conv2.w"):
        DevModel().prepare(m)
    with pytest.raises(om.FormatError, match="conv weight K not multiple of 9"):
        om.dev_model(om.parse_poisd(p.read_bytes()))
    m.close()
