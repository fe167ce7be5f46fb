"""Calls with no histories and no masks take the main pass's own kernel instance, whose parts may be twice as long
(131072 tokens) with a listing target and valve scaled to the part. Here a batch large enough to take them (512 rows,
two parts a row) over an odd vocabulary (150001 tokens: two parts of 75776 and 74225, a ragged tail), with a row stride
of V + 5 and a start two elements in (every other row not 16-byte aligned: both load paths in one launch), fp32 and bf16
logits, greedy and sampled rows with top-k, top-p, min-p, temperatures, ties and logprobs. The sampled tokens and the
logprob ids of a spread of rows are compared bit-exactly with the oracle, the logprobs within 1e-5."""
import numpy as np
import pytest
import torch

from oracle import sampling_ref as ora

pytestmark = pytest.mark.gpu

B, V, NLP = 512, 150001, 5
CHECK = [0, 1, 2, 3, 5, 8, 13, 64, 127, 255, 256, 300, 401, 510, 511]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_plain_call_long_parts(ge, gpu, dtype):
    g = torch.Generator(device=gpu)
    g.manual_seed(11)
    xd = torch.randn((B, V + 5), generator=g, device=gpu, dtype=torch.float32) * 2.0
    xd[7, 2:2 + 64] = 3.0                                  # ties at the top of one row
    xd[9, 2:2 + V] = 0.0                                   # a flat row
    if dtype == "bf16":
        xd = xd.to(torch.bfloat16)
    xt = xd[:, 2:2 + V]                                    # row stride V + 5, misaligned start
    P = ge.sampling.SamplingParams
    kinds = [P(temperature=1.0, logprobs=NLP), P(temperature=0.7, top_p=0.9), P(temperature=0.0, logprobs=NLP),
             P(temperature=1.3, top_k=50), P(temperature=0.9, min_p=0.05), P(temperature=1.0, top_p=0.95, top_k=400)]
    params = [kinds[r % len(kinds)] for r in range(B)]
    seeds, idxs = list(range(B)), [3] * B
    print(f"[plain parts] gse_sample over {B} x {V} {dtype}", flush=True)
    sel = ge.sampling.sample_ex(xt, params, seeds, idxs, None)
    torch.cuda.synchronize()
    got = np.array(sel.tolist())
    ids, lps = sel.logprob_ids.cpu().numpy(), sel.logprobs.cpu().numpy()

    xs = xt[CHECK].float().cpu().numpy()
    ps = [params[r] for r in CHECK]
    want = ora.sample_full(xs, ps, [seeds[r] for r in CHECK], [idxs[r] for r in CHECK], None, None, None)
    for k, r in enumerate(CHECK):
        assert got[r] == want[k]["token"], (r, got[r], want[k]["token"])
        if params[r].logprobs:
            assert list(ids[r][:NLP]) == list(want[k]["logprob_ids"]), r
            np.testing.assert_allclose(lps[r][:NLP], want[k]["logprobs"], rtol=1e-5, atol=1e-6)
