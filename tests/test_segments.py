"""CPU pins of long-audio segmentation (transcribe_audio, transcribe.rs:297-403)
and of the text rule with an opened text region.

- or_find_split_point (find_split_point, transcribe.rs:252-277) against a
  float64 brute force over the 1600-sample windows (hop 800) inside
  target +- search, and known answers: one silent window at an odd multiple
  of the hop (a wrong hop or window size lands elsewhere), two equal silent
  gaps (the first wins: strict `<`), no window inside the range (target);
- or_segment_splits (transcribe.rs:323-341): segment_sec <= 0 and audio
  within one segment plus the margin give [0]; the search radius is clamped
  to segment_sec / 2 (a silent gap just outside the clamp is not taken); at
  most 127 starts; starts never decrease and each lies within the search
  radius of its target;
- the library's qasr_hip_segment_splits (host code of the engine's
  transcribe_pcm) equals the oracle on random and edge inputs;
- qasr_hip_text_tokens_from: with text_open every token before the first
  stop except <asr_text> is text (past_asr_text starts true,
  transcribe.rs:196-214).
No GPU."""
import numpy as np
import pytest

SR, WIN, HOP = 16000, 1600, 800
ASR_TEXT, EOT, IM_END = 151704, 151643, 151645


def noise(n, seed, amp=0.1):
    return (np.random.default_rng(seed).standard_normal(n) * amp).astype(np.float32)


def brute_split(x, target, search_sec):
    """find_split_point in float64: (centers, energies) of every window."""
    half = int(np.float32(search_sec) * np.float32(SR)) if search_sec > 0 else 0
    lo, hi = max(target - half, 0), min(target + half, x.size)
    centers, energies = [], []
    pos = lo
    while pos + WIN <= hi:
        w = x[pos:pos + WIN].astype(np.float64)
        centers.append(pos + WIN // 2)
        energies.append(float(np.mean(w * w)))
        pos += HOP
    return centers, energies


def test_find_split_point_brute_force(orc):
    r = np.random.default_rng(11)
    for trial in range(60):
        n = int(r.integers(WIN, 40 * SR))
        x = (r.standard_normal(n) * r.uniform(0.001, 1.0, n)).astype(np.float32)
        target = int(r.integers(0, n))
        search = float(r.choice([0.05, 0.5, 1.0, 3.0, 7.5]))
        got = orc.find_split_point(x, target, search)
        centers, energies = brute_split(x, target, search)
        if not centers:
            assert got == target
            continue
        e = np.asarray(energies)
        best = int(np.argmin(e))
        if np.sum(e <= e[best] * (1 + 1e-5)) == 1:             # a clear minimum
            assert got == centers[best], (trial, got, centers[best])
        else:
            assert got in centers and e[centers.index(got)] <= e[best] * (1 + 1e-5)


def test_find_split_point_known_answers(orc):
    target, search = 20 * SR, 3.0
    lo = target - int(search * SR)
    x = noise(40 * SR, 1)
    gap = lo + 11 * HOP                                     # one window, odd multiple of the hop
    x[gap:gap + WIN] = 0
    assert orc.find_split_point(x, target, search) == gap + WIN // 2
    y = noise(40 * SR, 2)
    for g in (lo + 7 * HOP, lo + 31 * HOP):                 # two equal silent gaps: the first
        y[g:g + WIN] = 0
    assert orc.find_split_point(y, target, search) == lo + 7 * HOP + WIN // 2
    assert orc.find_split_point(x, target, 0.0) == target   # no window fits
    assert orc.find_split_point(x[:100], 50, 3.0) == 50     # audio shorter than a window


def test_segment_splits_known_answers(orc):
    x = noise(90 * SR, 3)
    assert orc.segment_splits(x, 0.0).tolist() == [0]
    assert orc.segment_splits(x, -5.0).tolist() == [0]
    assert orc.segment_splits(x[:23 * SR], 20.0).tolist() == [0]          # 20 s + 3 s margin
    assert len(orc.segment_splits(x[:23 * SR + 1], 20.0)) == 2
    # search clamped to segment_sec / 2 = 1 s: for the first split (target
    # 2 s) a silent window at 4 s lies outside the clamped radius (a 3 s
    # radius would take it)
    z = noise(12 * SR, 4)
    z[4 * SR - WIN // 2:4 * SR + WIN // 2] = 0
    s = orc.segment_splits(z, 2.0, search_sec=3.0)
    assert abs(int(s[1]) - 2 * SR) <= SR and s[1] != 4 * SR
    # with the full 3 s radius (segment 8 s) the same kind of gap is found
    w = noise(30 * SR, 5)
    w[10 * SR - WIN // 2:10 * SR + WIN // 2] = 0
    assert orc.segment_splits(w, 8.0, search_sec=3.0)[1] == 10 * SR
    # at most 127 starts
    assert len(orc.segment_splits(noise(200 * SR, 6), 1.0)) == 127


def test_segment_splits_properties(orc):
    r = np.random.default_rng(12)
    for _ in range(30):
        n = int(r.integers(0, 120 * SR))
        x = noise(n, int(r.integers(1 << 30)), amp=float(r.uniform(0.01, 1)))
        seg, search = float(r.uniform(0.5, 30)), float(r.uniform(0.0, 5))
        s = orc.segment_splits(x, seg, search)
        assert s[0] == 0 and len(s) <= 127
        assert np.all(np.diff(s) >= 0)
        rad = int(np.float32(min(search, seg / 2)) * np.float32(SR))
        tgt = int(np.float32(seg) * np.float32(SR))
        for a, b in zip(s[:-1], s[1:]):
            assert abs(int(b) - (int(a) + tgt)) <= rad


def test_library_segment_splits_equal_oracle(orc):
    from qwenasr_amd.model import segment_splits
    r = np.random.default_rng(13)
    cases = [(0, 20.0, 3.0), (100, 20.0, 3.0), (5 * SR, float("nan"), 3.0), (50 * SR, 10.0, float("nan")),
             (50 * SR, 1e-6, 3.0), (70 * SR, 20.0, 0.0), (70 * SR, 20.0, -1.0)]
    cases += [(int(r.integers(0, 90 * SR)), float(r.uniform(-1, 40)), float(r.uniform(-1, 8))) for _ in range(40)]
    for i, (n, seg, search) in enumerate(cases):
        x = (np.random.default_rng(i).standard_normal(n) * np.random.default_rng(i + 99).uniform(0, 1, n)).astype(
            np.float32)
        assert segment_splits(x, seg, search).tolist() == orc.segment_splits(x, seg, search).tolist(), (n, seg, search)


def text_rule(raw, text_open):
    out, past = [], text_open
    for t in raw:
        if t in (EOT, IM_END):
            break
        if t == ASR_TEXT:
            past = True
        elif past:
            out.append(t)
    return out


@pytest.mark.parametrize("raw", [[], [5, 6], [ASR_TEXT, 5], [5, ASR_TEXT, 6, IM_END, 7], [EOT, 1], [1, 2, 3]])
def test_text_tokens_open(raw):
    from qwenasr_amd.model import text_tokens
    for open_ in (False, True):
        assert text_tokens(np.array(raw, np.int32), text_open=open_).tolist() == text_rule(raw, open_)
