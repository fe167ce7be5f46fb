"""gse_sample_noalloc (the entry point that allocates nothing: a static per-GPU workspace) against gse_sample on the
same batches through the C ABI: tokens, logprobs and processed logits bit-exact, on two calls in a row (the second with
a smaller batch, so the static workspace keeps the first call's contents), and the size limit's error."""
import ctypes as C

import numpy as np
import pytest
import torch


def _out(lib, rows, v, nlp, dev):
    toks = torch.full((rows,), -7, dtype=torch.int32, device=dev)
    proc = torch.empty((rows, v), dtype=torch.float32, device=dev)
    o = lib.Out()
    o.size = C.sizeof(lib.Out)
    o.tokens = toks.data_ptr()
    o.processed, o.processed_ld = proc.data_ptr(), v
    keep = [toks, proc]
    if nlp:
        ids = torch.empty((rows, nlp), dtype=torch.int32, device=dev)
        lps = torch.empty((rows, nlp), dtype=torch.float32, device=dev)
        o.logprob_ids, o.logprobs, o.logprobs_ld = ids.data_ptr(), lps.data_ptr(), nlp
        keep += [ids, lps]
    return o, keep


def _both(ge, batch, gpu):
    lib = ge._lib
    x = torch.from_numpy(batch.logits).to(gpu)
    if batch.bf16:
        x = x.view(torch.bfloat16)
    masks = None if batch.masks is None else [torch.from_numpy(m) for m in batch.masks]
    h, x, code, dev, b, keep = ge.sampling._prepare(x, batch.params, None, None, masks, batch.history,
                                                     batch.uniforms)
    nlp = max([p.logprobs or 0 for p in batch.params] + [0])
    o1, k1 = _out(lib, batch.rows, batch.vocab, nlp, dev)
    h.ck(h.L.gse_sample(h.h, C.byref(b), C.byref(o1)), "gse_sample")
    o2, k2 = _out(lib, batch.rows, batch.vocab, nlp, dev)
    rc = h.L.gse_sample_noalloc(C.byref(b), C.byref(o2))
    assert rc == 0, (rc, h.L.gse_last_error(None))
    torch.cuda.synchronize()
    for a, c in zip(k1, k2):
        assert torch.equal(a, c)
    return k2[0].cpu().tolist()


@pytest.mark.gpu
def test_noalloc_matches_gse_sample_twice(ge, gpu):
    from oracle import sampling_ref as ora
    big = ge.workloads.c3(rows=list(range(32)))            # 32 x 151936, masks, histories, deep rows
    small = ge.workloads.c1()                              # 8 x 32000 after it
    t1 = _both(ge, big, gpu)
    t2 = _both(ge, small, gpu)
    assert t2 == ora.sample(small.logits_f32(), small.params, None, None, None, small.history, small.uniforms)
    assert len(t1) == 32 and min(t1) >= 0


def test_noalloc_rejects_batches_past_its_limit(ge):
    lib = ge._lib
    L = lib.bind()
    b = lib.Batch()
    b.size = C.sizeof(lib.Batch)
    b.rows, b.vocab, b.ld = lib.NOALLOC_ROWS + 1, 1000, 1000
    o = lib.Out()
    o.size = C.sizeof(lib.Out)
    assert L.gse_sample_noalloc(C.byref(b), C.byref(o)) == lib.E_CAPACITY
    assert b"at most 32 rows of at most 163840 tokens" in L.gse_last_error(None)
    b.rows, b.vocab, b.ld = 4, lib.NOALLOC_VOCAB + 1, lib.NOALLOC_VOCAB + 1
    assert L.gse_sample_noalloc(C.byref(b), C.byref(o)) == lib.E_CAPACITY


def test_noalloc_refuses_the_profile_flag(ge):
    """GSE_BATCH_PROFILE records host-allocated events on a handle; the entry point that allocates nothing refuses it
    (before it touches a device)."""
    lib = ge._lib
    L = lib.bind()
    b = lib.Batch()
    b.size = C.sizeof(lib.Batch)
    b.rows, b.vocab, b.ld = 4, 1000, 1000
    b.flags = lib.BATCH_PROFILE
    o = lib.Out()
    o.size = C.sizeof(lib.Out)
    assert L.gse_sample_noalloc(C.byref(b), C.byref(o)) == lib.E_UNSUPPORTED
    assert b"GSE_BATCH_PROFILE" in L.gse_last_error(None)
