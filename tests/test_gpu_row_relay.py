# SPDX-License-Identifier: MIT
"""GPU parity of the two-segment relay row pass for bfloat16 logits (row-pass
kind 5, forced, at vocabularies from 65544 up to 155648 entries; rows its
fixed-base table cannot take fold from memory) against the CPU oracle, bit
for bit on every decode output (tokens, parents, lengths, scores, final
scores, row logsumexp, NaN/+inf flags).

The cases cover: random shapes and options (EOS, extra EOS, min_length,
banned tokens, n-gram blocking, repetition penalty, per-example steps); a
partial last chunk; many rows per workgroup; rows off the table path (NaN of
either sign, +inf, maximum in (0, 1), every value negative, every value
-inf); rows whose values are mostly +-0, or with fewer positive values than
the shortlist holds; ties at the top past the survivor capacity; shortlist
sizes 0, 1, 3 and the largest (K = 64); the overlapped decode."""

import numpy as np
import pytest

from tests.cases import first_difference, make_case, to_bits

pytestmark = pytest.mark.gpu

_VOCABS = [65544, 70000, 100008, 128256, 131072, 131080, 151936, 153600]


@pytest.fixture
def stream(hip):
    """The relay row pass (kind 5), chosen explicitly."""
    prev = hip.lib.dbs_hip_set_row_pass(5)
    yield hip
    hip.lib.dbs_hip_set_row_pass(prev)


def _check(hip, oracle, xin, kw, label, **extra):
    want = oracle.decode(xin, dtype="bf16", **kw)
    got = hip.decode(xin, "bf16", **kw, **extra)
    diff = first_difference(got, want)
    assert diff is None, f"{label}: {diff}"
    return got


@pytest.mark.parametrize("seed", range(0, 16))
def test_stream_random_cases(stream, oracle, seed):
    case = make_case(13000 + seed, dtypes=["bf16"], vocabs=_VOCABS, logits=True, scales=[0.5, 2.0, 3.0, 8.0])
    kw = dict(case["kw"])
    _check(stream, oracle, case["xin"], kw, f"seed {seed} B{case['B']} T{case['T']} K{case['K']} V{case['V']}")


def _logits(rng, shape, V, scale=3.0):
    """Logits ~N(0, scale) plus a per-token Zipf bias shared across rows."""
    x = rng.normal(0.0, scale, size=shape + (V,)).astype(np.float32)
    x += (-1.1 * np.log(rng.permutation(V) + 1.0)).astype(np.float32)
    return x


def test_stream_many_rows_per_workgroup(stream, oracle):
    """1024 rows: several per workgroup, both LDS parities, tickets."""
    rng = np.random.default_rng(5)
    V = 65544
    x = _logits(rng, (2, 32, 16), V)
    kw = dict(from_logits=True, eos_token=V - 9, min_length=3, alpha=0.6)
    _check(stream, oracle, to_bits(x, "bf16"), kw, "1024 rows")


def test_stream_many_rows_largest_chunk_count(stream, oracle):
    """640 rows of 151936 entries (75 chunks of 2048, the last partial):
    several rows per workgroup with the chunk loads running across rows."""
    rng = np.random.default_rng(6)
    V = 151936
    x = _logits(rng, (2, 20, 16), V)
    kw = dict(from_logits=True, eos_token=V - 293, min_length=4, alpha=1.0)
    _check(stream, oracle, to_bits(x, "bf16"), kw, "640 rows V=151936")


def _special_rows(rng, V):
    """Rows that leave the streaming pass's common path."""
    rows = {}
    base = lambda: _logits(rng, (), V)
    r = base(); r[rng.integers(0, V)] = np.nan; rows["nan"] = r
    # a NaN with the sign bit set (patched into the bfloat16 bits below)
    r = base(); r[rng.integers(0, V)] = np.float32(123.0); rows["neg_nan"] = r
    r = base(); r[rng.integers(0, V)] = np.inf; rows["pos_inf"] = r
    r = base(); r[rng.random(V) < 0.3] = -np.inf; rows["some_neg_inf"] = r
    rows["max_below_one"] = (rng.random(V).astype(np.float32) * 0.9)
    rows["all_negative"] = -(rng.random(V).astype(np.float32) * 5.0 + 0.01)
    rows["all_neg_inf"] = np.full(V, -np.inf, np.float32)
    # threshold +0: zeros and -0 everywhere, a few values >= 1
    r = np.zeros(V, np.float32); r[rng.random(V) < 0.5] = -0.0
    r[rng.choice(V, 5, replace=False)] = [1.0, 2.0, 3.0, 4.0, 5.0]; rows["theta_zero"] = r
    # fewer than M threads hold a positive value (the threshold falls back to
    # the smallest positive value): lanes 0-2 of every stripe
    r = -(rng.random(V).astype(np.float32) + 0.5)
    idx = np.arange(V); r[(idx % 256) < 3] = 2.0 + rng.random(int(((idx % 256) < 3).sum())).astype(np.float32)
    rows["no_threshold"] = r
    # ties at the top past the survivor capacity
    r = base(); top = float(r.max()) + 1.0; r[rng.choice(V, 2000, replace=False)] = top; rows["top_ties"] = r
    # a top value in the last (partial) chunk and at token 0
    r = base(); r[V - 1] = r.max() + 3.0; r[0] = r[V - 1] - 0.5; rows["top_at_edges"] = r
    # huge and tiny magnitudes around the term table's edges
    r = base(); r[rng.choice(V, 64, replace=False)] = rng.choice([1e-30, -1e-30, 1e-40, -1e-40, 0.0, -0.0, -1e30], 64)
    rows["table_edges"] = r
    return rows


@pytest.mark.parametrize("V", [65544, 131080, 151936])
def test_stream_special_rows(stream, oracle, V):
    rng = np.random.default_rng(V)
    rows = _special_rows(rng, V)
    names = sorted(rows)
    # one example per row kind: step 0 ordinary, the row at step 1 beam 0
    # (K = 2: both beams of step 1 are read)
    x = np.stack([np.stack([_logits(rng, (2,), V), np.stack([rows[n], _logits(rng, (), V)])]) for n in names])
    x = x.astype(np.float32)
    assert x.shape == (len(names), 2, 2, V)
    xin = to_bits(x, "bf16")
    t = names.index("neg_nan")
    v = int(np.flatnonzero(x[t, 1, 0] == np.float32(123.0))[0])
    xin[t, 1, 0, v] = 0xff81
    kw = dict(from_logits=True, eos_token=V - 3, extra_eos=[5], min_length=2, alpha=1.0)
    got = _check(stream, oracle, xin, kw, f"V={V} rows {names}")
    want_invalid = [1 if n in ("nan", "neg_nan", "pos_inf") else 0 for n in names]
    assert got["invalid"].tolist() == want_invalid


@pytest.mark.parametrize("shortlist", ["0", "1", "3"])
def test_stream_shortlist_sizes(stream, oracle, shortlist, monkeypatch):
    monkeypatch.setenv("DBS_HIP_SHORTLIST", shortlist)
    rng = np.random.default_rng(int(shortlist) + 40)
    V = 131072
    x = _logits(rng, (2, 3, 4), V)
    kw = dict(from_logits=True, eos_token=17, min_length=1, alpha=0.6)
    _check(stream, oracle, to_bits(x, "bf16"), kw, f"shortlist {shortlist}")


@pytest.mark.parametrize("K", [1, 64, 100])
def test_stream_beam_widths(stream, oracle, K):
    """K = 1, the widest beam with a shortlist (K = 64, M = 80) and K > 64
    (no shortlist: every read row is rescanned)."""
    rng = np.random.default_rng(K + 300)
    V = 100008
    x = _logits(rng, (1, 2, K), V)
    kw = dict(from_logits=True, eos_token=2, min_length=0, alpha=1.0)
    _check(stream, oracle, to_bits(x, "bf16"), kw, f"K={K}")


def test_stream_banned_and_min_length(stream, oracle):
    """Banned tokens and EOS below min_length among the top values: the
    shortlist drops them and bounds the rest."""
    rng = np.random.default_rng(77)
    V = 151936
    x = _logits(rng, (2, 4, 8), V)
    top = np.argsort(-x.reshape(-1, V).max(axis=0))[:40]
    banned = np.zeros(V, np.uint8)
    banned[top[::2]] = 1
    kw = dict(from_logits=True, eos_token=int(top[1]), extra_eos=[int(top[3])], min_length=3, alpha=1.0,
              banned=banned, steps=[4, 2])
    _check(stream, oracle, to_bits(x, "bf16"), kw, "banned/min_length")


@pytest.mark.parametrize("overlap", [1, 0])
def test_stream_overlapped_select(stream, oracle, overlap):
    """The select pass running alongside the streaming row pass (rows
    published word by word) gives the same bits, with no wait given up."""
    import ctypes as C

    lib = stream.lib
    prev = lib.dbs_hip_set_decode_overlap(overlap)
    try:
        lib.dbs_hip_profile_enable(1)
        rng = np.random.default_rng(overlap + 90)
        V = 128256
        x = _logits(rng, (3, 6, 8), V)
        kw = dict(from_logits=True, eos_token=V - 11, min_length=4, alpha=1.0)
        _check(stream, oracle, to_bits(x, "bf16"), kw, f"overlap {overlap}")
        ms, n = C.c_double(), C.c_int64()
        assert lib.dbs_hip_profile_read(6, C.byref(ms), C.byref(n)) == 0
        assert n.value == 0, "a wait of the overlapped decode gave up"
    finally:
        lib.dbs_hip_profile_enable(0)
        lib.dbs_hip_set_decode_overlap(prev)
