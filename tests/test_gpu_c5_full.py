"""The large-vocabulary nucleus workload at its full size (B=1024, V=262144 bf16, top-p 0.9, top-20 logprobs) through
gse_sample in one call: rows the oracle generates and samples on the CPU are compared bit-exactly (tokens, logprob ids)
and within 1e-6 (logprobs); every row of the batch is checked against a torch fp64 restatement of the same draw
(sampling.py:59-85: stable descending order, fp64 softmax, the top-p prefix, the cumulative draw with the row's shared
uniform) and of the logprobs. The restatement sums in another order than numpy, so a row whose draw or top-p boundary
lies within 1e-9 of the total mass from a cumulative sum is counted as ambiguous and left to the bit-exact rows."""
import numpy as np
import pytest
import torch

from oracle import sampling_ref as ora

pytestmark = pytest.mark.gpu

B, V, NLP, TOP_P = 1024, 262144, 20, 0.9
ORACLE_ROWS = [0, 1, 2, 77, 511, 512, 900, 1023]


def _batch(ge, gpu):
    """Gumbel(0, 1) x 1.5 logits rounded to bf16 (torch's generator on the device for the bulk of the batch), with the
    oracle rows replaced by the workload generator's own rows."""
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    x = torch.empty((B, V), dtype=torch.bfloat16, device=gpu)
    for r0 in range(0, B, 128):
        u = torch.rand((128, V), dtype=torch.float64, device=gpu, generator=g).clamp_(1e-300, 1.0 - 1e-16)
        x[r0:r0 + 128] = (1.5 * -torch.log(-torch.log(u))).float().to(torch.bfloat16)
    sub = ge.workloads.c5(rows=ORACLE_ROWS)
    x[ORACLE_ROWS] = torch.from_numpy(sub.logits.view(np.int16)).to(gpu).view(torch.bfloat16)
    uni = ge.workloads.uniforms(3, np.arange(B, dtype=np.uint64))
    return x, uni, sub


def _torch_reference(x, uni):
    """Per row: the expected token, whether the row is ambiguous, and the top-NLP logprob ids and values."""
    toks, amb, lp_ids, lps = [], [], [], []
    for r0 in range(0, B, 64):
        z = x[r0:r0 + 64].float()
        zs, order = torch.sort(z, dim=1, descending=True, stable=True)
        zd = zs.double()
        e = torch.exp(zd - zd[:, :1])
        tot = e.sum(1, keepdim=True)
        q = e / tot
        cq = torch.cumsum(q, 1)
        keep = (cq - q) < TOP_P
        c = torch.cumsum(q * keep, 1)
        u = torch.from_numpy(uni[r0:r0 + 64]).to(x.device)[:, None]
        thr = u * c[:, -1:]
        j = torch.minimum((c < thr).sum(1), keep.sum(1) - 1).clamp_(min=0)
        toks.append(order.gather(1, j[:, None])[:, 0])
        # ambiguous: the draw threshold or the top-p boundary within 1e-9 of a prefix sum
        amb.append(((c - thr).abs() < 1e-9).any(1) | (((cq - q) - TOP_P).abs() < 1e-9).any(1))
        lp = (zd[:, :NLP] - zd[:, :1]) - torch.log(tot)
        lp_ids.append(order[:, :NLP])
        lps.append(lp.float())
    return (torch.cat(toks).cpu().numpy(), torch.cat(amb).cpu().numpy(), torch.cat(lp_ids).cpu().numpy(),
            torch.cat(lps).cpu().numpy())


def test_c5_full_batch(ge, gpu):
    x, uni, sub = _batch(ge, gpu)
    params = [ge.sampling.SamplingParams(temperature=1.0, top_p=TOP_P, logprobs=NLP) for _ in range(B)]
    print(f"[c5 full] gse_sample over {B} x {V} bf16", flush=True)
    sel = ge.sampling.sample_ex(x, params, None, None, None, uniforms=uni)
    torch.cuda.synchronize()
    got = np.array(sel.tolist())
    ids, lps = sel.logprob_ids.cpu().numpy(), sel.logprobs.cpu().numpy()
    paths = ge._lib.handle(gpu.index, B, V).row_paths(B)
    print(f"[c5 full] paths main/deep/exact: {[(paths == k).sum() for k in range(3)]}", flush=True)

    # the oracle's own rows: bit-exact tokens and logprob ids
    want = ora.sample_full(sub.logits_f32(), sub.params, None, None, None, None, sub.uniforms)
    for k, r in enumerate(ORACLE_ROWS):
        assert got[r] == want[k]["token"], (r, got[r], want[k]["token"])
        assert list(ids[r]) == list(want[k]["logprob_ids"]), r
        np.testing.assert_allclose(lps[r], want[k]["logprobs"], rtol=1e-6, atol=1e-6)

    # every row against the fp64 restatement
    tok_ref, amb, ref_ids, ref_lps = _torch_reference(x, uni)
    assert amb.sum() <= 4, amb.sum()
    bad = np.nonzero((got != tok_ref) & ~amb)[0]
    assert len(bad) == 0, (bad[:10], got[bad[:10]], tok_ref[bad[:10]])
    assert (ids == ref_ids).all(axis=1).sum() == B
    np.testing.assert_allclose(lps, ref_lps, rtol=1e-6, atol=1e-6)
    # properties: a token of the row, inside its nucleus (checked above through the reference), logprobs descending
    assert ((got >= 0) & (got < V)).all()
    assert (np.diff(lps, axis=1) <= 0).all()
