"""CPU models of the exact evaluations of a left-to-right f32 sum in
project-willamette_amd/csrc/wm_seqsum.h, in numpy float32, compared bit for
bit with the left-to-right float32 accumulation:

* the one-wave algorithm (64 lanes x 8 terms per step, the 128-term
  sequential lead, the run test on s's significand, restarts that zero
  consumed terms);
* the workgroup algorithm (binades predicted from a float64 prefix sum,
  break terms, integer segment sums, a sequential walk over the breaks with a
  check of every prediction and the one-wave algorithm on any segment whose
  check fails).

They check the algorithms themselves (exactness, the bound on passes per
step) without a GPU; the GPU tests check the device code against the same
sequential sums."""
import numpy as np
import pytest

f32 = np.float32
LANES, PER = 64, 8
STEP = LANES * PER
LEAD = 128


class PassCapReached(RuntimeError):
    pass


def _parity_increments(rr, half, N):
    """Increments of one pass with halfway terms resolved (PARITY): lane
    summaries (bit 1: the lane holds a halfway term; bit 0: parity of the
    increments after its last one, or of all of them), their inclusive
    segmented scan over the 64 lanes, one lane down, then each lane's terms
    in order, as wm::seq_sum_step<true> does."""
    rho = np.where(half, np.floor(rr), np.rint(rr)).astype(np.int64)
    summ = np.zeros(LANES, np.int64)
    for lane in range(LANES):
        x = 0
        for j in range(PER):
            x = 2 if half[lane, j] else x ^ (int(rho[lane, j]) & 1)
        summ[lane] = x

    def comb(left, right):
        return right if right & 2 else (left & 2) | ((left ^ right) & 1)

    incl = [0] * LANES
    acc = 0
    for lane in range(LANES):
        acc = comb(acc, int(summ[lane]))
        incl[lane] = acc
    out = rho.copy()
    for lane in range(LANES):
        xe = incl[lane - 1] if lane else 0
        par = (xe & 1) if xe & 2 else ((N ^ xe) & 1)
        for j in range(PER):
            if half[lane, j]:
                out[lane, j] += (par + int(rho[lane, j])) & 1
                par = 0
            else:
                par ^= int(rho[lane, j]) & 1
    return out


def model_sum(a, parity=False, stats=None):
    """Returns (sum, largest pass index used in any step).  parity: halfway
    terms are resolved by the segmented parity scan instead of ending a run.
    stats["passes"]: passes over all steps."""
    a = np.asarray(a, np.float32)
    n = a.size
    s = f32(0.0)
    max_pass = 0
    if n == 0:
        return s, 0
    buf = np.zeros(-(-n // STEP) * STEP, np.float32)
    buf[:n] = a
    pos = np.arange(STEP).reshape(LANES, PER)
    for k in range(0, n, STEP):
        v = buf[k:k + STEP].reshape(LANES, PER).copy()
        v[k + pos >= n] = 0
        if k == 0:
            with np.errstate(all="ignore"):
                for t in range(LEAD):
                    s = f32(s + v[t // PER, t % PER])
            v[:LEAD // PER, :] = 0
        for ps in range(STEP + 1):
            max_pass = max(max_pass, ps)
            if stats is not None:
                stats["passes"] = stats.get("passes", 0) + 1
            if np.isnan(s):
                return s, max_pass
            bits = int(np.array(s, np.float32).view(np.uint32))
            ef = bits >> 23
            normal = 1 <= ef <= 254
            sh = 150 - ef if normal else (255 if ef == 0 else -255)
            N = ((bits & 0x7FFFFF) | 0x800000) if normal else 0
            with np.errstate(all="ignore"):
                r = np.ldexp(v, sh).astype(np.float32)
            fin = r < f32(2.0 ** 22)
            rr = np.where(fin, r, f32(0)).astype(np.float32)
            half = (rr - np.floor(rr)) == f32(0.5)
            if parity:
                bad = ~fin
                rho = _parity_increments(rr, half, N)
            else:
                bad = (~fin) | half
                rho = np.rint(rr).astype(np.int64)
            p = np.cumsum(rho, axis=1)
            incl = np.cumsum(p[:, -1])
            excl = incl - p[:, -1]
            limit = (1 << 24) - 1 - N
            off = bad | ((rho > 0) & (excl[:, None] + p >= limit))
            if not off.any():
                if normal:
                    s = f32(np.ldexp(f32(N + int(incl[-1])), -sh))
                break
            fl, jl = divmod(int(np.argmax(off.reshape(-1))), PER)
            pre = int(excl[fl]) + (int(p[fl, jl - 1]) if jl else 0)
            if normal:
                s = f32(np.ldexp(f32(N + pre), -sh))
            with np.errstate(all="ignore"):
                s = f32(s + v[fl, jl])
            v[pos <= PER * fl + jl] = 0
        else:
            raise PassCapReached()
    return s, max_pass


WAVE_RECORDS = 96  # break records per wave the workgroup algorithm keeps (else: one-wave path)
BLOCK_THREADS = 1024


def _exp2floor(x):
    """floor(log2 x) of a positive finite float64."""
    return int(np.frexp(x)[1]) - 1


def _near_pow2(x, t):
    """x (positive, finite) within relative 2^-t of a power of two, by its bits."""
    mant = int(np.array(x, np.float64).view(np.uint64)) & ((1 << 52) - 1)
    return mant <= (1 << (52 - t)) or (1 << 52) - mant <= (1 << (53 - t))


def model_block_sum(a, stats=None, nt=BLOCK_THREADS, start_prefix=None, near_rule=True):
    """Model of wm::seq_sum_block_owned: returns the sum.

    Thread t owns terms t*m .. t*m+m-1 (m = ceil(n / nt)) and starts from a
    float64 prefix of the terms before them; `start_prefix(t, exact_prefix)`
    may return another value for it, standing for a different order of the
    same additions on the device (within relative 2^-45 of the exact one)."""
    a = np.asarray(a, np.float32)
    n = a.size
    if n == 0:
        return f32(0.0)
    m = -(-n // nt)
    with np.errstate(all="ignore"):
        S = np.concatenate([[0.0], np.cumsum(a.astype(np.float64))])  # S[k]: sum before term k
    waves = {}  # wave -> [(index, binade after, wave increments before, value)]
    wave_pi = {}
    for t in range(-(-n // m)):
        k0 = t * m
        w = t // 64
        P = S[k0]
        if start_prefix is not None and t > 0:
            P = start_prefix(t, P)
        recs = waves.setdefault(w, [])
        for k in range(k0, min(k0 + m, n)):
            v = a[k]
            pb = P
            with np.errstate(all="ignore"):
                pa = np.float64(P) + np.float64(v)
            P = pa
            pb_ok = 0 < pb < 1e300
            pa_ok = 0 < pa < 1e300
            zero = v == 0  # changes no running sum: never a break on its own account
            eb = _exp2floor(pb) if pb_ok else 0
            brk = not zero and (k == 0 or not pb_ok or not pa_ok or _exp2floor(pa) != eb)
            if near_rule:  # only where the prefix crosses a thread boundary
                brk = brk or (k == k0 and pb_ok and _near_pow2(pb, 34)) or \
                    (k == min(k0 + m, n) - 1 and pa_ok and _near_pow2(pa, 36))
            if not brk:
                with np.errstate(all="ignore"):
                    r = np.float32(np.ldexp(v, 23 - eb))
                brk = not (r < f32(2.0 ** 22)) or (r - np.floor(r)) == f32(0.5)
            if brk:
                ea = _exp2floor(pa) if pa_ok else -1000
                recs.append((k, ea, wave_pi.get(w, 0), v))
            else:
                wave_pi[w] = wave_pi.get(w, 0) + int(np.rint(r))
    if stats is not None:
        stats["breaks"] = sum(len(r) for r in waves.values())
        stats["max_wave_breaks"] = max((len(r) for r in waves.values()), default=0)
        stats["fallback_segments"] = 0
    if any(len(r) > WAVE_RECORDS for r in waves.values()):
        return model_sum(a)[0]
    # join the wave lists: global increment prefix = increments of earlier waves + wave-local
    recs, off = [], 0
    for w in sorted(set(waves) | set(wave_pi)):
        recs += [(k, ea, off + p, v) for (k, ea, p, v) in waves.get(w, [])]
        off += wave_pi.get(w, 0)
    s = f32(0.0)
    prev_t, prev_pi, e_seg = -1, 0, None
    for (t, ea, pit, v) in recs + [(n, None, off, None)]:
        cnt = t - prev_t - 1
        if cnt > 0 and prev_t < 0:
            # before the first break: zeros only (a non-zero term on a zero
            # prefix is a break), which add nothing
            assert not np.any(a[:t]), "non-zero term before the first break"
        elif cnt > 0:
            d = pit - prev_pi
            bits = int(np.array(s, np.float32).view(np.uint32))
            ef = bits >> 23
            ok = 1 <= ef <= 254 and e_seg is not None and ef - 127 == e_seg and 0 <= d <= (1 << 24)
            if ok:
                N = (bits & 0x7FFFFF) | 0x800000
                ok = N + d <= (1 << 24) - 2
            if ok:
                s = f32(np.ldexp(f32(N + d), e_seg - 23))
            else:  # the segment by the one-wave algorithm, from s
                if stats is not None:
                    stats["fallback_segments"] += 1
                with np.errstate(all="ignore"):
                    for x in a[prev_t + 1:t]:
                        s = f32(s + x)
        if t < n:
            with np.errstate(all="ignore"):
                s = f32(s + v)
            e_seg = ea
        prev_t, prev_pi = t, pit
    return s


def sequential(a):
    a = np.asarray(a, np.float32)
    if a.size == 0:
        return f32(0.0)
    with np.errstate(all="ignore"):
        return np.add.accumulate(a, dtype=np.float32)[-1]


def same(x, y):
    x, y = np.float32(x), np.float32(y)
    return (np.isnan(x) and np.isnan(y)) or x.view(np.uint32) == y.view(np.uint32)


def inputs():
    rng = np.random.default_rng(7)
    out = [
        ("empty", np.zeros(0, np.float32)),
        ("sq2560", rng.standard_normal(2560).astype(np.float32) ** 2),
        ("sq6912", rng.standard_normal(6912).astype(np.float32) ** 2),
        ("zeros", np.zeros(3000, np.float32)),
        ("subnormal", np.full(2000, 1e-40, np.float32)),
        ("ties_ulp2", np.concatenate([[2.0 ** 24], rng.integers(0, 4, 3000)]).astype(np.float32)),
        ("allones_significand", np.concatenate(
            [[16777215.0], np.zeros(LEAD - 1), [0.25, 0, 0, 1.0, 0.5, 3.0], np.ones(1000)]).astype(np.float32)),
        ("overflow", np.full(300, 3e37, np.float32)),
    ]
    x = (rng.standard_normal(1100) * 8).astype(np.float32)
    out.append(("softmax_wide", np.exp(x - x.max()).astype(np.float32)))
    nan = rng.standard_normal(700).astype(np.float32) ** 2
    nan[400] = np.nan
    out.append(("nan", nan))
    return out


@pytest.mark.parametrize("name,a", inputs(), ids=[c[0] for c in inputs()])
def test_model_matches_sequential(name, a):
    got, max_pass = model_sum(a)
    assert same(got, sequential(a)), name
    assert max_pass <= STEP


def test_model_fuzz():
    rng = np.random.default_rng(11)
    for i in range(400):
        n = int(rng.integers(1, 2000))
        sc = float(2.0 ** rng.integers(-20, 20))
        kind = i % 4
        if kind == 0:
            a = (rng.standard_normal(n) * sc).astype(np.float32) ** 2
        elif kind == 1:
            a = (rng.integers(0, 8, n) * sc).astype(np.float32)
        elif kind == 2:
            x = (rng.standard_normal(n) * 8).astype(np.float32)
            a = np.exp(x - x.max()).astype(np.float32)
        else:
            a = np.full(n, f32(2.0 ** rng.integers(-3, 3)), np.float32)
            a[0] = f32(2 ** 24 - 1) * f32(2.0 ** rng.integers(-30, 0))
        got, _ = model_sum(a)
        assert same(got, sequential(a)), f"case {i} kind {kind} n {n}"


@pytest.mark.parametrize("name,a", inputs(), ids=[c[0] for c in inputs()])
def test_parity_model_matches_sequential(name, a):
    got, max_pass = model_sum(a, parity=True)
    assert same(got, sequential(a)), name
    assert max_pass <= STEP


def test_parity_model_fuzz():
    rng = np.random.default_rng(12)
    for i in range(300):
        n = int(rng.integers(1, 2000))
        sc = float(2.0 ** rng.integers(-20, 20))
        kind = i % 3
        if kind == 0:  # coarse grids: most terms are halfway at some binade
            a = (rng.integers(0, 8, n) * sc).astype(np.float32)
        elif kind == 1:
            a = (rng.standard_normal(n) * sc).astype(np.float32) ** 2
        else:
            a = _q6k_like_squares(rng, n)
        got, _ = model_sum(a, parity=True)
        assert same(got, sequential(a)), f"case {i} kind {kind} n {n}"


def _parity_sequential(rr, half, N):
    """The increments of one pass evaluated term by term in sum order."""
    out = np.zeros(rr.shape, np.int64)
    par = N & 1
    for t in range(rr.size):
        lane, j = divmod(t, PER)
        if half[lane, j]:
            k = int(np.floor(rr[lane, j]))
            out[lane, j] = k + ((par + k) & 1)
            par = 0
        else:
            out[lane, j] = int(np.rint(rr[lane, j]))
            par ^= int(out[lane, j]) & 1
    return out


def test_parity_scan_matches_term_by_term():
    # the lane summaries and their segmented scan give every term the
    # increment a term-by-term evaluation gives (halfway terms on the even
    # neighbour of the running significand); sparse and dense halfway terms
    rng = np.random.default_rng(13)
    for i in range(200):
        k = rng.integers(0, 9, (LANES, PER)).astype(np.float32)
        half = rng.random((LANES, PER)) < [0.0, 0.02, 0.2, 0.6, 1.0][i % 5]
        rr = np.where(half, k + f32(0.5), k).astype(np.float32)
        N = int(rng.integers(1 << 23, 1 << 24))
        assert (_parity_increments(rr, half, N) == _parity_sequential(rr, half, N)).all(), i


def _q6k_like_squares(rng, n):
    """Squares of Q6_K-dequantised values as the embedding rows hold them:
    x = (d * sc) * q (d an f16 super-block scale, sc in [-32, 31] per 16
    elements, q in [-32, 31]); their few significant bits put many squares
    on halfway increments."""
    x = np.empty(n, np.float32)
    for b in range(0, n, 256):
        d = np.float32(np.float16(abs(rng.standard_normal()) * 1e-3))
        for c in range(b, min(b + 256, n), 16):
            dd = np.float32(d * np.float32(rng.integers(-32, 32)))
            q = rng.integers(-32, 32, min(16, n - c)).astype(np.float32)
            x[c:c + 16] = (dd * q).astype(np.float32)
    return (x * x).astype(np.float32)


def test_parity_cuts_passes_on_embedding_squares():
    # the rows of a step's first norm (some of them hold more than
    # WAVE_RECORDS breaks in one wave of a 512-thread norm and go to the
    # one-wave path): with halfway terms resolved in place a step needs far
    # fewer passes
    rng = np.random.default_rng(14)
    plain, par = {}, {}
    for _ in range(12):
        a = _q6k_like_squares(rng, 2560)
        got_p, _ = model_sum(a, parity=True, stats=par)
        got, _ = model_sum(a, stats=plain)
        assert same(got_p, sequential(a)) and same(got, sequential(a))
    assert 2 * plain["passes"] >= 3 * par["passes"], (plain, par)


def test_zero_increment_terms_never_end_a_run():
    # Without the increment guard, a consumed (zeroed) term satisfies the
    # crossing test when N = 2^24 - 1 and the pass repeats without progress.
    a = np.concatenate([[16777215.0], np.zeros(LEAD - 1), [0.25, 0, 0, 1.0]]).astype(np.float32)
    got, max_pass = model_sum(a)
    assert same(got, sequential(a)) and max_pass < 8


@pytest.mark.parametrize("name,a", inputs(), ids=[c[0] for c in inputs()])
def test_block_model_matches_sequential(name, a):
    assert same(model_block_sum(a), sequential(a)), name


def test_block_model_fuzz():
    rng = np.random.default_rng(13)
    fallbacks = 0
    for i in range(600):
        n = int(rng.integers(1, 7000))
        sc = float(2.0 ** rng.integers(-20, 20))
        kind = i % 5
        if kind == 0:
            a = (rng.standard_normal(n) * sc).astype(np.float32) ** 2
        elif kind == 1:
            a = (rng.integers(0, 8, n) * sc).astype(np.float32)
        elif kind == 2:
            x = (rng.standard_normal(n) * 8).astype(np.float32)
            a = np.exp(x - x.max()).astype(np.float32)
        elif kind == 3:
            a = np.full(n, f32(2.0 ** rng.integers(-3, 3)), np.float32)
            a[0] = f32(2 ** 24 - 1) * f32(2.0 ** rng.integers(-30, 0))
        else:  # sums that sit on binade boundaries
            a = np.full(n, f32(1.0), np.float32)
            a[::3] = f32(2.0) ** -rng.integers(20, 26)
        st = {}
        got = model_block_sum(a, st)
        if kind != 3:  # kind 3 makes every term a tie: the fallback is the point
            fallbacks += st["fallback_segments"]
        assert same(got, sequential(a)), f"case {i} kind {kind} n {n}"
    # predictions rarely fail on the other inputs
    assert fallbacks < 10


def test_block_model_rms_inputs_take_the_fast_path():
    rng = np.random.default_rng(3)
    for n in (2560, 6912):
        for _ in range(20):
            a = rng.standard_normal(n).astype(np.float32) ** 2
            st = {}
            assert same(model_block_sum(a, st), sequential(a))
            assert st["breaks"] < 64 and st["fallback_segments"] <= 2


def _boundary_case():
    """Terms whose exact prefix at a thread boundary (term 38, m = 2) is
    4096 - 2^-40, while the f32 running sum lags at 4096 - 3*2^-12: the
    terms 2^-14 ... 2^-40 round away in f32.  Then 2^-11 (2 ulps below 4096,
    1 ulp above), the tie 2^-12, and zeros."""
    head = [4096.0 - 3 * 2.0 ** -12] + [2.0 ** -14] * 11 + [2.0 ** -i for i in range(15, 41)]
    tail = [2.0 ** -11, 2.0 ** -12] + [0.0] * 1460
    return np.array(head + tail, np.float32)


def _flip_across_pow2(t, P):
    """Another order's value of a prefix: within relative 2^-45 of P, on the
    other side of a power of two whenever P is that close to one."""
    e = _exp2floor(P)
    for j in (e, e + 1):
        if abs(P - 2.0 ** j) <= 2.0 ** (j - 46):
            return 2.0 ** j * (1 + 2.0 ** -47) if P < 2.0 ** j else 2.0 ** j * (1 - 2.0 ** -47)
    return P


def test_block_model_boundary_prefix_order():
    """A thread's prefix computed in another order may land on the other
    side of a power of two than the previous thread's running prefix.
    The near-power-of-two breaks keep the sum exact; without them the
    segment's increments are taken in two different binades."""
    a = _boundary_case()
    assert -(-a.size // BLOCK_THREADS) == 2
    want = sequential(a)
    assert same(model_block_sum(a, start_prefix=_flip_across_pow2), want)
    assert not same(model_block_sum(a, start_prefix=_flip_across_pow2, near_rule=False), want)


def test_block_model_boundary_fuzz():
    """Random prefixes pushed across nearby powers of two at every thread start."""
    rng = np.random.default_rng(17)
    for i in range(200):
        n = int(rng.integers(1025, 7000))
        m = -(-n // BLOCK_THREADS)
        a = rng.integers(1, 4, n).astype(np.float32)
        # make some thread boundary sit just below or at a power of two
        k = m * int(rng.integers(1, n // m))
        pre = float(np.sum(a[:k], dtype=np.float64))
        target = 2.0 ** (int(np.log2(pre)) + 1)
        a[k - 1] = np.float32(a[k - 1] + (target - pre) - rng.choice([0.0, 2.0 ** -20]))
        if not np.isfinite(a).all() or (a < 0).any():
            continue
        assert same(model_block_sum(a, start_prefix=_flip_across_pow2), sequential(a)), f"case {i}"


def _softmax_underflow(rng, n, live):
    """exp(s - max) of scores whose spread underflows all but the last `live`
    terms to exactly zero (a softmax dominated by the newest positions)."""
    s = np.concatenate([rng.standard_normal(n - live) * 4.0 - 200.0, rng.standard_normal(live) * 3.0])
    e = np.exp((s - s.max()).astype(np.float32)).astype(np.float32)
    assert (e[: n - live] == 0).all()
    return e


def test_block_model_zero_runs_are_not_breaks():
    """Zero terms change no running sum, so runs of them (a zero prefix, an
    underflowed softmax tail) cost no breaks; the sum stays exact."""
    rng = np.random.default_rng(23)
    cases = [np.zeros(1088, np.float32), _softmax_underflow(rng, 1088, 64),
             _softmax_underflow(rng, 4000, 5), _softmax_underflow(rng, 2049, 1)]
    sparse = (rng.standard_normal(3000) ** 2).astype(np.float32)
    sparse[rng.random(3000) < 0.9] = 0.0
    cases.append(sparse)
    lead = np.concatenate([np.zeros(700), rng.random(388) + 0.5]).astype(np.float32)
    cases.append(lead)
    for i, a in enumerate(cases):
        st = {}
        assert same(model_block_sum(a, st), sequential(a)), f"case {i}"
        nz = int(np.count_nonzero(a))
        # breaks come from the non-zero terms (binade changes, the first
        # non-zero term) and the rare near-power-of-two boundaries
        assert st["breaks"] <= min(nz, 64) + 4, f"case {i}: {st['breaks']} breaks, {nz} non-zero"


def test_block_model_zero_runs_fuzz():
    rng = np.random.default_rng(29)
    for i in range(200):
        n = int(rng.integers(1, 4096))
        a = (rng.standard_normal(n) ** 2 * 2.0 ** rng.integers(-30, 30)).astype(np.float32)
        a[rng.random(n) < rng.random()] = 0.0
        assert same(model_block_sum(a), sequential(a)), f"case {i}"


def _thread_breaks_full(P, v, k0, last):
    """One thread's (break, increment, binade after a break) per term by the
    full test of wm::seq_sum_block_owned (every ok check, k == 0, zero
    terms); the binade is recorded, and used, only at breaks."""
    out = []
    with np.errstate(all="ignore"):
        for j, x in enumerate(v):
            k = k0 + j
            pb, pa = P, np.float64(P) + np.float64(x)
            P = pa
            pb_ok, pa_ok = 0 < pb < 1e300, 0 < pa < 1e300
            eb = _exp2floor(pb) if pb_ok else 0
            ea = _exp2floor(pa) if pa_ok else -1000
            b = x != 0 and (k == 0 or not pb_ok or not pa_ok or ea != eb)
            b = b or (j == 0 and pb_ok and _near_pow2(pb, 34))
            b = b or (j == last and pa_ok and _near_pow2(pa, 36))
            d = 0
            if not b:
                r = np.float32(np.ldexp(np.float32(x), 23 - eb))
                b = not (r < f32(2.0 ** 22)) or (r - np.floor(r)) == f32(0.5)
                d = 0 if b else int(np.rint(r))
            brk = bool(j <= last and b)
            out.append((brk, d if j <= last else 0, ea if brk else None))
    return out


def _binade_field(x):
    """The device's exp2floor_f64: the biased exponent field minus 1023 (-1023 for +0)."""
    return int((int(np.array(x, np.float64).view(np.uint64)) >> 52) & 0x7FF) - 1023


def _thread_breaks_posfin(P, v, last):
    """The same by the device's shortcut for a thread whose prefix chain
    ends finite: one binade comparison per term, no ok checks."""
    with np.errstate(all="ignore"):
        Pe = P
        for x in v:
            Pe = np.float64(Pe) + np.float64(x)
        assert Pe < 1e300
        close0 = P > 0 and _near_pow2(P, 34)
        close1 = Pe > 0 and _near_pow2(Pe, 36)
        eb = _binade_field(P)
        out = []
        for j, x in enumerate(v):
            P = np.float64(P) + np.float64(x)
            ea = _binade_field(P)
            b = (x != 0 and ea != eb) or (j == 0 and close0) or (j == last and close1)
            r = np.float32(np.ldexp(np.float32(x), 23 - eb))
            b = b or not (r < f32(2.0 ** 22)) or (r - np.floor(r)) == f32(0.5)
            brk = bool(j <= last and b)
            out.append((brk, int(np.rint(r)) if j <= last and not b else 0, ea if brk else None))
            eb = ea
    return out


def test_positive_prefix_shortcut_matches_full_test():
    """A thread whose float64 prefix chain stays finite gets the same breaks,
    increments and binades from the shortcut as from the full test:
    prefixes that start at zero (the first term of the sum, leading zeros),
    cross powers of two or sit next to one, terms that are ties, zeros,
    subnormal or too large for a run."""
    rng = np.random.default_rng(11)
    cases = 0
    for _ in range(3000):
        m = int(rng.integers(1, 17))
        kind = rng.integers(0, 5)
        if kind == 0:  # squares of N(0,1)
            v = (rng.standard_normal(m).astype(np.float32) ** 2).astype(np.float32)
        elif kind == 1:  # wide exponents, some zeros and subnormals
            v = np.ldexp(rng.random(m), rng.integers(-150, 40, m)).astype(np.float32)
            v[rng.random(m) < 0.3] = 0
        elif kind == 2:  # small integers: ties and exact sums
            v = rng.integers(0, 9, m).astype(np.float32) * f32(0.5)
        elif kind == 3:  # a term far above the prefix
            v = rng.random(m).astype(np.float32)
            v[rng.integers(0, m)] = f32(2.0 ** 40)
        else:  # powers of two
            v = np.ldexp(np.ones(m), rng.integers(-10, 10, m)).astype(np.float32)
        # a starting prefix near a power of two, or anywhere
        e = int(rng.integers(-20, 30))
        P = float(np.ldexp(1.0, e)) * (1 + float(rng.choice([0.0, 2.0 ** -40, -(2.0 ** -40), rng.random()])))
        if rng.random() < 0.2:
            P = float(np.ldexp(1.0, e)) - float(v.astype(np.float64).sum()) * float(rng.random())
        k0 = int(rng.integers(1, 10000))
        if rng.random() < 0.15:  # the first thread, or one inside a run of leading zeros
            P, k0 = 0.0, int(rng.choice([0, k0]))
            if rng.random() < 0.5:
                v[: int(rng.integers(0, m + 1))] = 0
        if not P >= 0:
            continue
        last = int(rng.integers(0, m)) if rng.random() < 0.3 else m - 1
        v[last + 1:] = 0  # terms past the last valid one are zeros on the device
        assert _thread_breaks_posfin(P, v, last) == _thread_breaks_full(P, v, k0, last)
        cases += 1
    assert cases > 2500


def test_round_clamp_fast_formula():
    """wm_round_clamp_i8_fast: min(trunc_sat_u32(|v|) + (fract(|v|) >= 0.5),
    127) with v's sign equals wm_round_clamp_i8 (round half away from zero,
    clamp to +-127, NaN -> 0) on a dense sample of float bit patterns, every
    value next to a half-integer in range, and the special values."""
    def reference(v):
        with np.errstate(all="ignore"):
            r = np.where(np.abs(v - np.trunc(v)) >= 0.5, np.trunc(v) + np.sign(v), np.trunc(v))
            r = np.clip(r, -127, 127)
        return np.where(np.isnan(r), 0, r).astype(np.int64)

    def fast(v):
        with np.errstate(all="ignore"):
            a = np.abs(v).astype(np.float64)
            # v_cvt_u32_f32: truncate, NaN -> 0, saturate to [0, 2^32 - 1]
            u = np.where(np.isnan(a), 0, np.minimum(np.trunc(a), 2.0 ** 32 - 1))
            fract = a - np.floor(a)  # v_fract_f32 (NaN for inf and NaN)
            u = u + np.where(fract >= 0.5, 1, 0)
        m = np.minimum(u.astype(np.int64), 127)
        return np.where(np.signbit(v), -m, m)

    bits = np.arange(0, 2 ** 32, 251, dtype=np.uint64).astype(np.uint32)
    halves = np.arange(-140, 141, dtype=np.float64) + 0.5
    near = np.concatenate([np.nextafter(halves.astype(np.float32), np.float32(np.inf)),
                           np.nextafter(halves.astype(np.float32), np.float32(-np.inf)),
                           halves.astype(np.float32), np.arange(-140, 141, dtype=np.float32)])
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 2.0 ** 22, 2.0 ** 23, 2.0 ** 24,
                        127.49999, 127.5, -127.5, 1e-45, -1e-45, 3e38, -3e38,
                        0.49999997, -0.49999997, 0.5, -0.5], np.float32)
    for v in (bits.view(np.float32), near, special):
        assert np.array_equal(fast(v), reference(v))
