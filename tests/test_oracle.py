"""CPU tests that pin the oracle: golden vectors from the reference, closed forms,
invariants and planted mistakes (a plausible error planted in the oracle must make
one of the pins fail)."""
import os

import numpy as np
import pytest

from oracle import delta_oracle as O
from oracle import select_oracle_c as OC

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "hybrid_golden.npz")


def _golden(case):
    z = np.load(GOLDEN)
    g = lambda n: z[f"{case}/{n}"]
    return {n: g(n) for n in ("q", "k", "v", "keep", "window", "no_count",
                             "out_hybrid", "out_sanity", "out_pure_phase1")}


def _run_golden(case, variant, fn=O.hybrid_attention):
    d = _golden(case)
    p = O.pack(d["k"], d["v"], d["keep"])
    out = fn(d["q"], d["k"], d["v"], p["k_packed"], p["v_packed"], p["timestamps"], p["counts"],
             int(d["window"]), variant=variant, no_count=bool(d["no_count"]))
    return out, d[f"out_{variant}"]


# --------------------------------------------------------------------------------------
# golden vectors written by the reference's own kernels
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["A", "B", "C", "D"])
@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1"])
def test_oracle_matches_reference_golden(case, variant):
    out, ref = _run_golden(case, variant)
    assert np.abs(out - ref).max() < 1e-5


@pytest.mark.parametrize("case", ["A", "B"])
@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1"])
def test_bruteforce_matches_reference_golden(case, variant):
    out, ref = _run_golden(case, variant, O.hybrid_bruteforce)
    assert np.abs(out - ref).max() < 1e-5


def test_golden_cases_cover_the_quirks():
    """Case A double counts (Phase 1 and Phase 2 both run), case B hits the padding-block
    reset (a fully padded safe block sets ds back to 0), case C is no_count with W = 0."""
    d = _golden("A")
    p = O.pack(d["k"], d["v"], d["keep"])
    ns, last, ds, _ = O.hybrid_schedule(p["timestamps"], p["P"], 1000, 1000, 128)
    assert (ns > 0).any() and (ds[ns > 0] <= last[ns > 0]).all()
    d = _golden("B")
    p = O.pack(d["k"], d["v"], d["keep"])
    ns, last, ds, _ = O.hybrid_schedule(p["timestamps"], p["P"], 640, 640, 128)
    assert ns[0, 0, -1] == 3 and last[0, 0, -1] == 0 and ds[0, 0, -1] == 0
    assert bool(_golden("C")["no_count"])


def _planted(monkeypatch, mutate):
    real = O.hybrid_schedule

    def wrong(ts, P, n_k, n_q, window):
        n_safe, last, ds, dh = real(ts, P, n_k, n_q, window)
        return mutate(n_safe, last, ds, dh)
    monkeypatch.setattr(O, "hybrid_schedule", wrong)


@pytest.mark.parametrize("mistake", ["no_double_count", "ds_from_last", "stop_one_early",
                                     "ignore_padding_reset"])
def test_planted_schedule_mistakes_fail_golden(monkeypatch, mistake):
    """Each plausible misreading of deltaFlashAttention.py:66-109, planted in the oracle,
    makes the golden comparison fail."""
    def mutate(n_safe, last, ds, dh):
        if mistake == "no_double_count":      # Phase 2 starts after the last packed block
            ds = np.where(n_safe > 0, np.maximum(ds, n_safe * 0 + ((last + 1 + 127) // 128) * 128), ds)
        elif mistake == "ds_from_last":       # (last // 128) * 128 instead of (last + 1)
            ds = np.maximum(0, (last // 128) * 128)
        elif mistake == "stop_one_early":
            n_safe = np.maximum(0, n_safe - 1)
        elif mistake == "ignore_padding_reset":  # treat padded blocks as unsafe
            ds = np.where((last == 0) & (n_safe > 1), 128, ds)
        return n_safe, last, ds, dh
    _planted(monkeypatch, mutate)
    worst = 0.0
    for case in "ABC":
        out, ref = _run_golden(case, "hybrid")
        worst = max(worst, float(np.abs(out - ref).max()))
    # the keep-all invariant (hybrid == dense) pins the "+1" of (last + 1) // 128, which
    # only matters when last is 127 mod 128 -- always the case when every row is an anchor
    q, k, v = _layer()
    p = O.pack(k, v, np.ones(k.shape[:3], np.int32))
    out = O.hybrid_attention(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"], 0)
    worst = max(worst, float(np.abs(out - O.dense_bruteforce(q, k, v)).max()))
    assert worst > 1e-3, f"planted mistake {mistake} went unnoticed"


def test_planted_count_mistake_fails_golden(monkeypatch):
    """Dropping the count weighting (counts -> 1) is caught by the golden vectors."""
    real = O.hybrid_attention

    def wrong(*a, **kw):
        kw["no_count"] = True
        return real(*a, **kw)
    out, ref = _run_golden("A", "hybrid", wrong)
    assert np.abs(out - ref).max() > 1e-3


# --------------------------------------------------------------------------------------
# selection: closed forms
# --------------------------------------------------------------------------------------
def _collinear(N, step, chunk):
    k = np.zeros((1, 1, N, 128), np.float32)
    k[0, 0, :, 0] = (np.arange(N) % chunk) * step
    return k


@pytest.mark.parametrize("impl", [O.select_delta, OC.select_delta])
@pytest.mark.parametrize("tau,period", [(1.5, 4), (2.0, 5), (0.25, 1)])
def test_select_collinear_closed_form(impl, tau, period):
    """Rows on a line with step 0.5: dist^2 to the anchor a is ((i - a) / 2)^2, so a row is
    kept iff i - a > 2 tau (strict); anchors repeat every `period` rows from each chunk
    start.  tau = 2 puts row a + 4 exactly on the threshold, which must not be kept."""
    N, chunk = 1100, 512
    keep, counts = impl(_collinear(N, 0.5, chunk), tau, chunk)
    want = np.zeros(N, np.int32)
    for s in range(0, N, chunk):
        want[s:min(s + chunk, N):period] = 1
    assert (keep[0, 0] == want).all()
    assert (counts[0, 0] == [want[s:s + chunk].sum() for s in range(0, N, chunk)]).all()


@pytest.mark.parametrize("impl", [O.select_delta, OC.select_delta])
def test_select_constant_keys_keep_chunk_starts(impl):
    k = np.ones((1, 2, 1000, 64), np.float32)
    keep, counts = impl(k, 0.0, 100)
    assert keep.sum() == 2 * 10 and (keep[:, :, ::100] == 1).all()
    assert (counts == 1).all()


@pytest.mark.parametrize("impl", [O.select_delta, OC.select_delta])
def test_select_cosine_on_a_circle(impl):
    """Keys rotate by theta per row: cos to the anchor is cos((i - a) theta); with tau
    between cos(3 theta) and cos(4 theta) every 4th row is an anchor."""
    N, theta = 600, 0.1
    ang = np.arange(N) * theta
    k = np.zeros((1, 1, N, 128), np.float32)
    k[0, 0, :, 0], k[0, 0, :, 1] = np.cos(ang), np.sin(ang)
    tau = 0.5 * (np.cos(3 * theta) + np.cos(4 * theta))
    keep, _ = impl(k, tau, 512, 0, "cosine")
    want = np.zeros(N, np.int32)
    want[0:512:4] = 1
    want[512::4] = 1
    assert (keep[0, 0] == want).all()


def test_select_metric_string_rule():
    """Only the exact string "cosine" is cosine (modeling_llama.py:639-640)."""
    rng = np.random.default_rng(0)
    k = rng.standard_normal((1, 1, 300, 128)).astype(np.float32)
    a = O.select_delta(k, 15.0, 512, 0, "euclidean")[0]
    for name in ("cos", "euclidian", "Cosine"):
        assert (O.select_delta(k, 15.0, 512, 0, name)[0] == a).all()


def test_chunking_rules():
    assert O.chunking(1050, 100) == (100, 11)
    assert O.chunking(300, 512) == (300, 1)
    assert O.chunking(10, 0, 4) == (3, 4)
    assert O.chunking(3, 0, 5) == (1, 5)
    assert O.chunking(7, 0, 0) == (7, 1)
    keep, counts = O.select_delta(np.random.default_rng(1).standard_normal((1, 1, 3, 64)).astype(np.float32),
                                  0.0, 0, 5)
    assert counts.tolist() == [[[1, 1, 1, 0, 0]]]


def test_tree_sum_order_is_pairwise():
    """The fixed reduction is a pairwise tree: (1e8 + 1) + (-1e8 + 1) rounds to 0 in fp32,
    while a left-to-right sum gives 1."""
    x = np.zeros(128, np.float32)
    x[:4] = [1e8, 1.0, -1e8, 1.0]
    assert O.tree_sum(x) == 0.0
    x = np.zeros(128, np.float32)
    x[0], x[64] = 1e8, 1.0        # meet only at the root
    x[1] = -1e8
    assert O.tree_sum(x) == 1.0


@pytest.mark.parametrize("metric,tau", [("euclidean", 9.0), ("cosine", 0.85), ("euclidean", 3.0)])
def test_select_numpy_equals_c(metric, tau):
    rng = np.random.default_rng(7)
    e = rng.standard_normal((2, 2, 1200, 128)).astype(np.float32)
    k = np.empty_like(e)
    k[:, :, 0] = e[:, :, 0]
    for t in range(1, 1200):
        k[:, :, t] = 0.9 * k[:, :, t - 1] + 0.44 * e[:, :, t]
    k = O.bf16_round(k)
    a = O.select_delta(k, tau, 300, 0, metric)
    b = OC.select_delta(k, tau, 300, 0, metric)
    assert (a[0] == b[0]).all() and (a[1] == b[1]).all()


# --------------------------------------------------------------------------------------
# index / pack / counts: integer closed forms
# --------------------------------------------------------------------------------------
def test_pack_closed_forms():
    rng = np.random.default_rng(3)
    B, H, N, D = 2, 3, 700, 16
    k = rng.standard_normal((B, H, N, D)).astype(np.float32)
    v = rng.standard_normal((B, H, N, D)).astype(np.float32)
    keep = (rng.random((B, H, N)) < 0.3).astype(np.int32)
    keep[..., 0] = 1
    p = O.pack(k, v, keep)
    c = keep.sum(-1)
    assert p["P"] == c.max() and (p["anchor_counts"] == c).all()
    for b in range(B):
        for h in range(H):
            n = c[b, h]
            ts = p["timestamps"][b, h, :n]
            assert (np.diff(ts) > 0).all() and ts[0] == 0
            assert (p["k_packed"][b, h, :n] == k[b, h, ts]).all()
            assert (p["v_packed"][b, h, :n] == v[b, h, ts]).all()
            runs = np.diff(np.append(ts, N))
            assert (p["counts"][b, h, :n] == runs).all()           # run lengths
            assert p["counts"][b, h].sum() == N                     # every row counted once
            assert (p["counts"][b, h, n:] == 0).all() and (p["timestamps"][b, h, n:] == 0).all()
            assert (p["k_packed"][b, h, n:] == 0).all()
    assert (O.index_map(keep)[keep == 1] == np.concatenate(
        [np.arange(x) for x in c.ravel()])).all()


def test_periodic_rounding_is_bankers():
    """period = max(1, round(1/rate)) with Python's round: 1/0.4 = 2.5 -> 2."""
    keep = O.select_periodic(1, 1, 10, 0.4)
    assert keep[0, 0].tolist() == [1, 0, 1, 0, 1, 0, 1, 0, 1, 0]


# --------------------------------------------------------------------------------------
# attention invariants
# --------------------------------------------------------------------------------------
def _layer(N=640, Hq=4, Hkv=2, D=32, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((1, Hq, N, D)).astype(np.float32)
    k = rng.standard_normal((1, Hkv, N, D)).astype(np.float32)
    v = rng.standard_normal((1, Hkv, N, D)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("W", [0, 128])
def test_keep_all_hybrid_is_dense(W):
    q, k, v = _layer()
    keep = np.ones(k.shape[:3], np.int32)
    p = O.pack(k, v, keep)
    dense = O.dense_bruteforce(q, k, v)
    for fn in (O.hybrid_attention, O.hybrid_bruteforce):
        out = fn(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"], W)
        assert np.abs(out - dense).max() < 1e-5
    pure = O.hybrid_attention(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"],
                              W, variant="pure_phase1")
    assert np.abs(pure - dense).max() < 1e-5


def test_window_beyond_sequence_is_dense():
    q, k, v = _layer(N=500)
    keep, _ = O.select_delta(k, 6.0, 128)
    p = O.pack(k, v, keep)
    out = O.hybrid_attention(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"], 500)
    assert np.abs(out - O.dense_bruteforce(q, k, v)).max() < 1e-5


def test_pure_phase1_equals_repeated_keys():
    """A count-c anchor weighs exactly like c copies of its key (count-weighted softmax)."""
    q, k, v = _layer(N=384, Hq=2, Hkv=1)
    keep, _ = O.select_delta(k, 7.0, 128)
    p = O.pack(k, v, keep)
    out = O.hybrid_attention(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"],
                             128, variant="pure_phase1")
    n = p["anchor_counts"][0, 0]
    rep_k = np.repeat(p["k_packed"][0, 0, :n], p["counts"][0, 0, :n], axis=0)
    rep_v = np.repeat(p["v_packed"][0, 0, :n], p["counts"][0, 0, :n], axis=0)
    rep_t = np.repeat(p["timestamps"][0, 0, :n], p["counts"][0, 0, :n])
    for h in range(2):
        s = q[0, h] @ rep_k.T * 32 ** -0.5
        s = np.where(rep_t[None, :] <= np.arange(384)[:, None], s, -np.inf)
        e = np.exp(s - s.max(1, keepdims=True))
        ref = e @ rep_v / e.sum(1, keepdims=True)
        assert np.abs(out[0, h] - ref).max() < 1e-5


def test_dense_oracle_is_textbook_softmax():
    q, k, v = _layer(N=300, Hq=6, Hkv=3)
    for causal in (True, False):
        a = O.dense_attention(q, k, v, causal)
        b = O.dense_bruteforce(q, k, v, causal)
        assert np.abs(a - b).max() < 1e-5


# --------------------------------------------------------------------------------------
# decode: constructed sequences and identities
# --------------------------------------------------------------------------------------
def _decode_state(B, H, D, cap, W):
    return {"k_packed": np.zeros((B, H, cap, D), np.float32), "v_packed": np.zeros((B, H, cap, D), np.float32),
            "counts": np.zeros((B, H, cap), np.int32), "timestamps": np.zeros((B, H, cap), np.int32),
            "lengths": np.zeros(B * H, np.int32), "k_exact": np.zeros((B, H, W, D), np.float32),
            "v_exact": np.zeros((B, H, W, D), np.float32), "exact_len": 0, "total_len": 0, "window": W}


def test_decode_update_merge_append_sequence():
    """Keys on a line with step 1 and tau 2.5: an evicted key merges into the last packed
    key while its distance is <= 2.5 (strict > appends), so the packed cache keeps every
    3rd evicted token with count 3; counts plus ring occupancy account for every token."""
    W, T, D = 4, 30, 8
    st = _decode_state(1, 1, D, 64, W)
    for t in range(T):
        kk = np.zeros((1, 1, 1, D), np.float32)
        kk[..., 0] = t
        O.decode_update(st, kk, kk * 2, 2.5)
    n = int(st["lengths"][0])
    evicted = T - W
    assert st["counts"][0, 0, :n].sum() == evicted
    assert st["timestamps"][0, 0, :n].tolist() == list(range(0, evicted, 3))
    assert st["k_packed"][0, 0, :n, 0].tolist() == list(range(0, evicted, 3))
    assert st["counts"][0, 0, :n].tolist()[:-1] == [3] * (n - 1)
    assert sorted(st["k_exact"][0, 0, :, 0].tolist()) == list(range(T - W, T))


def test_decode_attention_log_count_identity():
    """exp(s + log c) = c exp(s): a count-c packed key equals c ring copies."""
    rng = np.random.default_rng(5)
    D, W = 16, 3
    st = _decode_state(1, 1, D, 8, W)
    st["k_packed"][0, 0, :3] = rng.standard_normal((3, D))
    st["v_packed"][0, 0, :3] = rng.standard_normal((3, D))
    st["counts"][0, 0, :3] = [1, 4, 2]
    st["lengths"][0] = 3
    st["k_exact"][0, 0] = rng.standard_normal((W, D))
    st["v_exact"][0, 0] = rng.standard_normal((W, D))
    st["exact_len"] = 10
    q = rng.standard_normal((1, 2, D)).astype(np.float32)
    out = O.decode_attention(q, st)
    keys = np.concatenate([np.repeat(st["k_packed"][0, 0, :3], [1, 4, 2], axis=0), st["k_exact"][0, 0]])
    vals = np.concatenate([np.repeat(st["v_packed"][0, 0, :3], [1, 4, 2], axis=0), st["v_exact"][0, 0]])
    for h in range(2):
        s = keys @ q[0, h] * D ** -0.5
        e = np.exp(s - s.max())
        assert np.abs(out[0, h] - e @ vals / e.sum()).max() < 1e-5


def test_decode_update_cosine_on_a_circle():
    """Cosine merge (deltaDecoding.py:67-72): evicted keys rotate by theta per token, so
    cos to the last packed key is cos((t - a) theta); with tau between cos(2 theta) and
    cos(3 theta) every third evicted token is appended."""
    W, T, D, theta = 3, 40, 8, 0.2
    st = _decode_state(1, 1, D, 64, W)
    tau = 0.5 * (np.cos(2 * theta) + np.cos(3 * theta))
    for t in range(T):
        kk = np.zeros((1, 1, 1, D), np.float32)
        kk[..., 0], kk[..., 1] = np.cos(t * theta), np.sin(t * theta)
        O.decode_update(st, kk, kk, tau, "cosine")
    n = int(st["lengths"][0])
    assert st["timestamps"][0, 0, :n].tolist() == list(range(0, T - W, 3))
    assert st["counts"][0, 0, :n].sum() == T - W


# --------------------------------------------------------------------------------------
# bf16 rounding (oracle.bf16_round) and the round_p paths that use it
# --------------------------------------------------------------------------------------
def test_bf16_round_matches_torch():
    """bf16_round against torch's own float32 -> bfloat16 conversion (round to nearest,
    ties to even) on values across the whole exponent range, exact ties with even and
    odd bf16 mantissas, overflow to infinity, signed zeros, infinities, NaN and
    subnormals.  A truncating or ties-away implementation fails the tie cases."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    n = 200000
    mant = rng.standard_normal(n)
    with np.errstate(over="ignore"):  # a few land beyond the float32 range: +-inf
        x = (mant * np.exp2(rng.integers(-150, 128, n).astype(np.float64))).astype(np.float32)
    bits = rng.integers(0, 1 << 32, 50000, dtype=np.uint64).astype(np.uint32)
    ties = ((bits & np.uint32(0xFFFF0000)) | np.uint32(0x8000)).view(np.float32)
    near = ((bits & np.uint32(0xFFFF0000)) | np.uint32(0x7FFF)).view(np.float32)
    special = np.array([1.00390625, 1.01171875, -1.00390625, -1.01171875, 0.0, -0.0, np.inf,
                        -np.inf, np.nan, 1e-40, -1e-40, 1e-45, 3.3961776e38, -3.3961776e38,
                        np.finfo(np.float32).max, np.finfo(np.float32).tiny, 0.7, 0.702],
                       dtype=np.float32)
    allv = np.concatenate([x, ties, near, special])
    got = O.bf16_round(allv)
    want = torch.from_numpy(allv.copy()).to(torch.bfloat16).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # the tie cases really are ties and go both ways
    r = O.bf16_round(ties[np.isfinite(ties)])
    up = np.abs(r) > np.abs(ties[np.isfinite(ties)])
    assert 0.3 < up.mean() < 0.7


def _round_p_case():
    """Two keys, scale 128**-0.5: row 1 scores key 0 at 0 and key 1 at ln(0.702), so
    p = (1, 0.702 +- 1e-7); bf16(0.702) = 0.703125 (round to nearest, unambiguous: the
    neighbours are 0.69921875 and 0.703125).  V = (0, 1) in dim 0."""
    D = 128
    scale = np.float32(D ** -0.5)
    q = np.zeros((1, 1, 2, D), np.float32)
    q[0, 0, 1, 0] = np.float32(np.log(0.702) / scale)
    k = np.zeros((1, 1, 2, D), np.float32)
    k[0, 0, 1, 0] = 1.0
    v = np.zeros((1, 1, 2, D), np.float32)
    v[0, 0, 1, 0] = 1.0
    p1 = float(np.exp(np.float32(q[0, 0, 1, 0] * scale)))
    return q, k, v, scale, p1


def test_round_p_hybrid_closed_form():
    """With round_p the P.V product takes bf16(p) while l keeps the fp32 p, as
    deltaFlashAttention.py:86-98 (p.to(v.dtype)); without it, p itself."""
    q, k, v, scale, p1 = _round_p_case()
    ts = np.zeros((1, 1, 1), np.int32)
    cnt = np.ones((1, 1, 1), np.int32)
    kp, vp = k[:, :, :1], v[:, :, :1]
    for round_p, num in ((True, 0.703125), (False, p1)):
        out = O.hybrid_attention(q, k, v, kp, vp, ts, cnt, window=1000, scale=scale, round_p=round_p)
        assert abs(out[0, 0, 1, 0] - num / (1.0 + p1)) < 1e-6, (round_p, out[0, 0, 1, 0])
        assert out[0, 0, 0, 0] == 0.0


def test_round_p_decode_closed_form():
    """decode_attention's round_p: one query, a packed anchor with count 1 scoring 0 and a
    ring key scoring ln(0.702)."""
    q, k, v, scale, p1 = _round_p_case()
    D = 128
    st = {"k_packed": k[:, :, :1].copy(), "v_packed": v[:, :, :1].copy(),
          "counts": np.ones((1, 1, 1), np.int32), "lengths": np.ones(1, np.int32),
          "k_exact": k[:, :, 1:].copy(), "v_exact": v[:, :, 1:].copy(), "exact_len": 1, "window": 1}
    for round_p, num in ((True, 0.703125), (False, p1)):
        out = O.decode_attention(q[:, :, 1], st, scale=scale, round_p=round_p)
        assert out.shape == (1, 1, D)
        assert abs(out[0, 0, 0] - num / (1.0 + p1)) < 1e-6, (round_p, out[0, 0, 0])


# --------------------------------------------------------------------------------------
# the torch-CPU baseline (bench.py's cpu_baseline leg) computes the oracle's attention
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["A", "B", "D"])
def test_cpu_baseline_hybrid_matches_golden(case):
    """The blockwise exact softmax over each block's weighted key multiset reproduces the
    reference's own kernels' outputs (double counting and the padding reset included)."""
    from oracle import cpu_baseline as CB
    d = _golden(case)
    if bool(d["no_count"]):
        pytest.skip("the baseline times the counted hybrid variant")
    p = O.pack(d["k"], d["v"], d["keep"])
    out = CB.hybrid_attention(d["q"], d["k"], d["v"], p["k_packed"], p["v_packed"], p["timestamps"],
                              p["counts"], int(d["window"])).numpy()
    assert np.abs(out - d["out_hybrid"]).max() < 1e-5


@pytest.mark.parametrize("N,Hq,Hkv,W,tau", [(700, 8, 2, 128, 6.0), (384, 4, 4, 0, 7.5), (1000, 4, 1, 300, 5.0)])
def test_cpu_baseline_matches_oracle(N, Hq, Hkv, W, tau):
    from oracle import cpu_baseline as CB
    q, k, v = _layer(N=N, Hq=Hq, Hkv=Hkv)
    keep, _ = O.select_delta(k, tau, 128)
    p = O.pack(k, v, keep)
    want = O.hybrid_attention(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"], W)
    got = CB.hybrid_attention(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"], W).numpy()
    assert np.abs(got - want).max() < 1e-5
    for causal in (True, False):
        got_d = CB.dense_attention(q, k, v, causal).numpy()
        assert np.abs(got_d - O.dense_bruteforce(q, k, v, causal)).max() < 1e-5


def test_cpu_baseline_keep_all_is_dense():
    from oracle import cpu_baseline as CB
    q, k, v = _layer(N=512, Hq=4, Hkv=2)
    p = O.pack(k, v, np.ones(k.shape[:3], np.int32))
    got = CB.hybrid_attention(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"], 128).numpy()
    assert np.abs(got - O.dense_bruteforce(q, k, v)).max() < 1e-5
