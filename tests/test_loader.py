"""`.tns` ingest: hand-written fixtures with known answers.

Pins the oracle's order-3 loader (oracle/cptc_oracle.cpp, tensor.cu:24-271)
and checks the product loaders (cptc_tns_load3, cptc_tns_probe_nmodes,
cptc_tns_load_generic; generic.cu:971-1155) against the same answers.  Pure
host code: runs without a GPU.
"""
import numpy as np
import pytest

# (text, expected (m0, m1, m2, val), expected dims) for the order-3 parser
CASES3 = [
    # comments, tabs, scientific notation
    ("# comment line\n1 1 1 1.5\n2 3 4 -2.25e1\n\t3\t2\t1\t7\n",
     ([0, 1, 2], [0, 2, 1], [0, 3, 0], [1.5, -22.5, 7.0]), (3, 3, 4)),
    # 0-based index maps to 0, blank line, last line without newline
    ("0 0 5 1\n\n1 2 3 2.5", ([0, 0], [0, 1], [4, 2], [1.0, 2.5]), (1, 2, 5)),
    # a line with three fields and no value is skipped
    ("1 2 3\n4 5 6 7.0\n", ([3], [4], [5], [7.0]), (4, 5, 6)),
    # CRLF: strtod skips '\r\n' and reads the next line's first field
    ("1 2 3\r\n4 5 6 7.0\r\n", ([0, 3], [1, 4], [2, 5], [4.0, 7.0]), (4, 5, 6)),
    # unparsable value skipped
    ("1 2 3 abc\n2 2 2 3\n", ([1], [1], [1], [3.0]), (2, 2, 2)),
    # indented '#' line: no digits anywhere -> strtod fails -> skipped
    ("  # x 1 2\n1 1 1 1\n", ([0], [0], [0], [1.0]), (1, 1, 1)),
    # a leading sign is not an index digit: indices parse as 0, value = -1
    ("-1 2 3 4\n", ([0], [0], [0], [-1.0]), (1, 1, 1)),
]


def _write(tmp_path, text, name="t.tns"):
    p = tmp_path / name
    p.write_bytes(text.encode())
    return str(p)


@pytest.mark.parametrize("text,exp,dims", CASES3)
def test_oracle_load3_known_answers(tmp_path, orc, text, exp, dims):
    m0, m1, m2, v, d = orc.load_tns3(_write(tmp_path, text))
    assert m0.tolist() == exp[0] and m1.tolist() == exp[1] and m2.tolist() == exp[2]
    assert v.tolist() == exp[3]
    assert tuple(d) == dims


@pytest.mark.parametrize("text,exp,dims", CASES3)
def test_product_load3_known_answers(tmp_path, ca, text, exp, dims):
    t = ca.load_tns3(_write(tmp_path, text))
    assert t.idx[0].tolist() == exp[0] and t.idx[1].tolist() == exp[1]
    assert t.idx[2].tolist() == exp[2]
    assert t.val.tolist() == exp[3]
    assert tuple(t.dims) == dims


def test_load3_missing_file(ca, orc, tmp_path):
    with pytest.raises(ca.CptcError):
        ca.load_tns3(str(tmp_path / "nope.tns"))
    with pytest.raises(RuntimeError):
        orc.load_tns3(str(tmp_path / "nope.tns"))


def test_load3_roundtrip_large(tmp_path, ca, orc):
    """Writer -> product loader -> oracle loader agree on a multi-chunk file."""
    t = ca.synth_zipf((300, 200, 500), (1.1, 1.1, 1.1), 300000, 0, 3)
    path = str(tmp_path / "big.tns")
    ca.write_tns(path, t)
    u = ca.load_tns3(path)
    m0, m1, m2, v, d = orc.load_tns3(path)
    assert np.array_equal(u.idx, t.idx) and np.array_equal(u.val, t.val)
    assert np.array_equal(np.stack([m0, m1, m2]).astype(np.uint32), t.idx)
    assert np.array_equal(v, t.val)
    assert tuple(u.dims) == tuple(d) == tuple(int(x) + 1 for x in t.idx.max(axis=1))


CASESN = [
    # header comment, order 4 (5 fields), dims = max 1-based index
    ("# hdr\n1 2 3 4 5.0\n2 1 1 1 1e-3\n", 4,
     [[0, 1], [1, 0], [2, 0], [3, 0]], [5.0, 0.001], (2, 2, 3, 4)),
    # 0-based input: index 0 -> 0, dims from the raw maximum (max 1 -> dim 1)
    ("0 0 0 1\n3 1 2 2\n", 3, [[0, 2], [0, 0], [0, 1]], [1.0, 2.0], (3, 1, 2)),
    # a short line is skipped
    ("1 1 1 1\n2 2\n3 3 3 3\n", 3, [[0, 2], [0, 2], [0, 2]], [1.0, 3.0], (3, 3, 3)),
]


@pytest.mark.parametrize("text,order,idx,val,dims", CASESN)
def test_product_load_generic_known_answers(tmp_path, ca, text, order, idx, val, dims):
    path = _write(tmp_path, text)
    assert ca.probe_nmodes(path) == order
    t = ca.load_tns_generic(path)
    assert t.idx.tolist() == idx
    assert t.val.tolist() == val
    assert tuple(t.dims) == dims


def test_probe_nmodes_missing_and_order3(tmp_path, ca):
    assert ca.probe_nmodes(str(tmp_path / "missing.tns")) == -1
    assert ca.probe_nmodes(_write(tmp_path, "\n# c\n1 2 3 4.0\n")) == 3


def test_long_lines(tmp_path, ca):
    """The N-order loader reads through a 4 MiB line buffer and aborts on a
    longer line (generic.cu:1132-1138); the order-3 loader reads lines of any
    length (std::getline, tensor.cu)."""
    pad = " " * (5 << 20)
    path = str(tmp_path / "long.tns")
    with open(path, "w") as f:
        f.write("1 2 3 4.0\n2" + pad + " 1 1 2.5\n")
    with pytest.raises(ca.CptcError, match="line longer than read buffer"):
        ca.load_tns_generic(path)
    t = ca.load_tns3(path)
    assert t.dims == (2, 2, 3) and list(t.val) == [4.0, 2.5]
    short = str(tmp_path / "short.tns")
    with open(short, "w") as f:
        f.write("1 2 3 4.0\n2" + " " * (3 << 20) + " 1 1 2.5\n")
    g = ca.load_tns_generic(short)
    assert g.dims == (2, 2, 3) and list(g.val) == [4.0, 2.5]


def test_generic_rejects_order1(tmp_path, ca):
    with pytest.raises(ca.CptcError):
        ca.load_tns_generic(_write(tmp_path, "1 2.0\n2 3.0\n"))


# Value spellings that strtod reads in its own ways; the loaders take plain
# decimals through a faster correctly-rounded parser and must give strtod's
# double for every one (Python's float() and the oracle's strtod agree on
# the plain ones; the others are written out).
VALUE_CASES = [
    ("1.5", 1.5), ("-0", -0.0), ("-.25", -0.25), (".5", 0.5), ("1.", 1.0), ("007.5", 7.5),
    ("1e5", 1e5), ("1E-5", 1e-5), ("2.5e+3", 2500.0), ("1.5e", 1.5), ("1e400", float("inf")),
    ("-1e400", float("-inf")), ("1e-400", 0.0), ("4.9406564584124654e-324", 5e-324),
    ("2.2250738585072011e-308", 2.2250738585072011e-308),
    ("0.1000000000000000055511151231257827", 0.1), ("123456789012345678901234567890", 1.2345678901234568e29),
    ("+3.5", 3.5), ("0x1p3", 8.0), ("0X10", 16.0), ("inf", float("inf")), ("-Infinity", float("-inf")),
    ("1.7976931348623157e308", 1.7976931348623157e308), ("9007199254740993", 9007199254740992.0),
]


@pytest.mark.parametrize("load", ["load3", "generic"])
def test_value_spellings_match_strtod(tmp_path, ca, orc, load):
    text = "".join(f"{i + 1} 1 1 {s}\n" for i, (s, _) in enumerate(VALUE_CASES))
    path = _write(tmp_path, text)
    t = ca.load_tns3(path) if load == "load3" else ca.load_tns_generic(path)
    _, _, _, ov, _ = orc.load_tns3(path)                 # the oracle: strtod itself
    exp = np.array([v for _, v in VALUE_CASES])
    assert np.array_equal(t.val, exp) and np.array_equal(np.signbit(t.val), np.signbit(exp))
    assert np.array_equal(t.val.view(np.uint64), np.asarray(ov).view(np.uint64))


def test_random_decimals_bit_exact(tmp_path, ca, orc):
    """Shortest round-trip spellings of log-normal doubles, as the synthetic
    generators write them, and truncated 6- to 20-digit spellings."""
    rng = np.random.default_rng(7)
    vals = np.concatenate([rng.lognormal(0.0, 3.0, 3000), -rng.lognormal(0.0, 30.0, 1000)])
    strs = [repr(float(x)) for x in vals]
    strs += [f"{x:.{d}g}" for x, d in zip(vals[:2000], rng.integers(6, 21, 2000))]
    text = "".join(f"1 1 {i + 1} {s}\n" for i, s in enumerate(strs))
    path = _write(tmp_path, text)
    t = ca.load_tns3(path)
    _, _, _, ov, _ = orc.load_tns3(path)
    assert t.val.view(np.uint64).tolist() == np.asarray(ov).view(np.uint64).tolist()
    assert t.val.tolist() == [float(s) for s in strs]
