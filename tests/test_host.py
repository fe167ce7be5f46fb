"""Host logic of the drop-in modules, without a GPU: parameter validation (sampling.py:23-39 plus the extensions),
the host integer helpers, the per-row record packing, mask packing, the synthetic workloads, and that the product path
refuses to run (no CPU fallback) when there is no HIP device."""
import numpy as np
import pytest
import torch

from oracle import sampling_ref as ora


def test_validate(ge):
    P = ge.sampling.SamplingParams
    for bad in (P(temperature=-1), P(top_p=0), P(top_k=-1), P(max_tokens=0), P(n=2), P(stop_sequences=((),)),
                P(accept="x"), P(repetition_penalty=0.0), P(frequency_penalty=float("inf")), P(min_p=1.5),
                P(min_p=-0.1), P(logprobs=65)):
        with pytest.raises(ValueError):
            bad.validate()
    P(temperature=0.7, top_k=5, top_p=0.9, min_p=0.05, repetition_penalty=1.2, frequency_penalty=-0.5,
      presence_penalty=0.3, logprobs=20).validate()


def test_mix_uniform_equal_the_oracle(ge):
    rng = np.random.default_rng(0)
    for _ in range(200):
        s, i = int(rng.integers(0, 2 ** 63)), int(rng.integers(0, 2 ** 40))
        assert ge.sampling.mix(s, i) == ora.mix(s, i)
        assert ge.sampling.uniform(s, i) == ora.uniform(s, i)
    idx = np.arange(100, dtype=np.uint64)
    assert (ge.workloads.mix_array(12345, idx) == ora.mix_np(12345, idx)).all()
    assert np.array_equal(ge.workloads.uniforms(3, idx), ora.uniform_np(3, idx))


def test_row_records(ge):
    P = ge.sampling.SamplingParams
    ps = [P(), P(temperature=1e-50, top_k=7, top_p=0.9, min_p=0.05, repetition_penalty=1.1, logprobs=3),
          P(temperature=0.8, top_k=10 ** 12)]
    r = ge.sampling._rows(ps, [1, 2 ** 64 + 5, None], [0, 9, 3], np.array([0, 2, 2, 5]))
    assert r["temperature"].tolist() == [0.0, 0.0, np.float32(0.8)]
    assert r["flags"].tolist() == [0, ge._lib.ROW_TEMP_UNDERFLOW, 0]   # positive t whose float32 is 0 is sampled
    assert r["top_k"].tolist() == [0, 7, 0x7FFFFFFF]
    assert r["seed"].tolist() == [1, 5, 0] and r["idx"].tolist() == [0, 9, 3]
    assert r["hist_begin"].tolist() == [0, 2, 2] and r["hist_end"].tolist() == [2, 2, 5]
    assert r["repetition_penalty"][1] == np.float32(1.1) and r["logprobs"].tolist() == [0, 3, 0]


class _PackedMatcher:
    """A matcher with xgrammar's packed fill (fill_next_token_bitmask(bitmask, index) writes row index)."""

    def __init__(self, ge, mask):
        self.words = ge.grammar.pack(mask)

    def fill_bitmask(self, buf, row):
        buf[row, :self.words.numel()] = self.words


def test_mask_batch_fill_and_rows(ge):
    """grammar.MaskBatch: matcher fills and set() give the packed words of each row; unfilled rows carry no mask;
    sample()'s mask step maps filled rows onto the batch's rows (here on the CPU device: no copy kernel involved)."""
    rng = np.random.default_rng(2)
    n, v = 6, 1000
    masks = [rng.random(v) < 0.4 for _ in range(n)]
    mb = ge.grammar.MaskBatch(n, v, pin=False)
    assert mb.host.shape == (n, (v + 31) // 32) and not mb.filled.any()
    mb.fill(0, _PackedMatcher(ge, masks[0]))
    mb.set(2, masks[2])                               # bool [V]
    mb.set(3, ge.grammar.pack(masks[3]))              # packed int32 words
    mb.set(5, torch.from_numpy(masks[5]))             # bool tensor
    assert mb.filled.tolist() == [True, False, True, True, False, True]
    for i in (0, 2, 3, 5):
        assert (mb.host[i].numpy() == ora.pack_mask(masks[i])).all()
    with pytest.raises(ValueError):
        mb.set(1, np.ones(v - 1, dtype=bool))
    params = [ge.sampling.SamplingParams() for _ in range(n)]
    rows = ge.sampling._rows(params, None, None, None)
    words, ld = ge.sampling._masks(None, mb, n, v, torch.device("cpu"), rows)
    assert ld == (v + 31) // 32 and words.shape == (n, ld)
    assert rows["mask_row"].tolist() == [0, -1, 2, 3, -1, 5]
    assert torch.equal(words, mb.host)
    with pytest.raises(ValueError):
        ge.sampling._masks(None, mb, n + 1, v, torch.device("cpu"), ge.sampling._rows(params + params[:1], None,
                                                                                        None, None))
    mb.reset()
    rows = ge.sampling._rows(params, None, None, None)
    assert ge.sampling._masks(None, mb, n, v, torch.device("cpu"), rows) == (None, 0)
    assert rows["mask_row"].tolist() == [-1] * n


def test_grammar_pack_unpack(ge):
    rng = np.random.default_rng(1)
    for v in (1, 31, 32, 33, 1000, 4097):
        m = rng.random(v) < 0.3
        w = ge.grammar.pack(m)
        assert w.shape == ((v + 31) // 32,)
        assert (ge.grammar.unpack(w, v).numpy() == m).all()
        assert (ora.unpack_mask(w.numpy(), v) == m).all()
        assert (w.numpy() == ora.pack_mask(m)).all()
        assert (ge.workloads.pack_bits(m[None])[0] == ora.pack_mask(m)).all()


def test_workloads_are_seeded_and_row_independent(ge):
    a = ge.workloads.c1()
    b = ge.workloads.c1(rows=[3, 5])
    assert a.logits.shape == (8, 32000) and a.logits.dtype == np.float32
    assert np.array_equal(a.logits[[3, 5]], b.logits) and np.array_equal(a.uniforms[[3, 5]], b.uniforms)
    assert abs(float(a.logits.std()) - 2.0) < 0.02
    c = ge.workloads.c3(rows=[0, 1])
    assert c.masks.shape == (2, 4748) and c.logits.shape == (2, 151936) and len(c.history[0]) == 2048
    allowed = ora.unpack_mask(c.masks[0], 151936)
    assert 0.02 < allowed.mean() < 0.08 and ora.unpack_mask(c.masks[1], 151936).all()
    assert abs(float(c.logits[0].mean())) < 1e-3
    p = c.params[0]
    assert 0.5 <= p.temperature <= 1.5 and p.top_k in (0, 20, 50, 200) and 0.8 <= p.top_p <= 1.0
    e = ge.workloads.c5(rows=[0])
    assert e.logits.dtype == np.uint16 and e.bf16
    f = ge.workloads.bf16_bits_to_f32(e.logits)
    assert np.isfinite(f).all() and abs(float(np.median(f)) - 1.5 * -np.log(np.log(2.0))) < 0.02   # Gumbel median


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the behaviour without a HIP device")
def test_product_path_refuses_without_a_gpu(ge):
    P = ge.sampling.SamplingParams
    x = np.zeros((1, 10), np.float32)
    with pytest.raises(RuntimeError):
        ge.sampling.sample(x, [P()], [0], [0], [None])
    with pytest.raises(RuntimeError):
        ge.sampling.draw(np.ones(4) / 4, 0.5)


def _least_ge_brute(t, S):
    """The least float64 x >= 0 with x / S >= t, by stepping one ulp at a time from far below (plain Python floats)."""
    import math
    x = max(0.0, t * S * (1 - 1e-12))
    while not (x / S >= t):
        x = math.nextafter(x, math.inf)
    while x > 0.0 and math.nextafter(x, 0.0) / S >= t:
        x = math.nextafter(x, 0.0)
    return x


def test_division_threshold_lies_within_eight_ulps():
    """The split-row finish replaces each test x / S >= t (x the exact fixed-point prefix as a double, S the row's mass,
    t = top_p, min_p q_0 or u c_last) by x >= a, with a the least double for which the test holds: RN(x / S) is
    non-decreasing in x, so that is the same test. The device finds a among the 16 doubles RN(t S) - 8 ulp ..
    RN(t S) + 7 ulp (one per lane) and sends the row to the exact path when they do not bracket it. Brute force over
    random and edge (t, S) here: a always lies in that window, and the window's first passing candidate is a."""
    import math
    rng = np.random.default_rng(11)
    cases = [(0.0, 1.0), (1.0, 1.0), (1.0, 151936.0), (0.9, 3.0), (1e-300, 2.0), (0.5, 2.0 ** 18), (1.0, 1.0 + 2 ** -52)]
    cases += [(float(rng.random()), float(1.0 + rng.random() * 2 ** 18)) for _ in range(3000)]
    cases += [(float(rng.random() * 1e-6), float(1.0 + rng.random() * 10)) for _ in range(500)]
    for t, S in cases:
        want = _least_ge_brute(t, S)
        x0 = t * S
        bits0 = np.float64(x0).view(np.int64)
        cand = [float(np.int64(max(b, 0)).view(np.float64)) if b > 0 else 0.0 for b in (bits0 + np.arange(-8, 8))]
        ok = [c / S >= t for c in cand]
        f = ok.index(True) if any(ok) else 16
        assert f < 16 and (f > 0 or cand[f] == 0.0), (t, S)
        assert cand[f] == want, (t, S, cand[f], want)
        assert all(ok[f:]) and not any(ok[:f]), (t, S)
        for x in (want, math.nextafter(want, 0.0), math.nextafter(want, math.inf)):
            assert (x / S >= t) == (x >= want)
