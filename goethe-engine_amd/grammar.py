"""Drop-in for goethe_engine/grammar.py: the same compiler / matcher surface, with the mask kept in xgrammar's packed
int32 form (token t allowed iff bit t % 32 of word t // 32 is set, LSB first; grammar.py:42-45) so that gse_sample
applies it on the GPU inside the fused pass instead of a host bool[V] unpack per row.

Matcher: mask() -> bool tensor [vocab] (as the reference); bitmask() -> int32 tensor [ceil(vocab / 32)] (packed, what
sample() consumes without unpacking); fill_bitmask(buf, row) writes the packed words into row `row` of an int32
[rows, ceil(vocab / 32)] buffer; accept(tok) -> bool; done() -> bool.
MaskBatch: the packed masks of one step's rows in one host buffer (pinned when a GPU is present) that sample() takes
as its masks argument and sends to the device in one copy.
Compiler: compile(kind, spec) -> object with new_matcher(). kind is "json_schema", "regex", "ebnf" or "json".
xgrammar is imported only when a compiler is built (it is not installed in every environment).
"""
import numpy as np
import torch


class XGrammarCompiler:
    def __init__(self, vocab, eos_ids=(), vocab_size=None):
        import xgrammar as xgr
        self.xgr, self.vocab_size = xgr, vocab_size or len(vocab)
        info = xgr.TokenizerInfo(vocab, vocab_size=self.vocab_size, stop_token_ids=list(eos_ids))
        self.c = xgr.GrammarCompiler(info)
        self.cache = {}

    def compile(self, kind, spec):
        key = (kind, spec)
        if key not in self.cache:
            c = self.c
            try:
                g = {"json_schema": lambda: c.compile_json_schema(spec), "regex": lambda: c.compile_regex(spec),
                     "ebnf": lambda: c.compile_grammar(spec), "json": c.compile_builtin_json_grammar}[kind]()
            except Exception as e:
                raise ValueError(f"grammar does not compile: {e}") from e
            self.cache[key] = _Compiled(self.xgr, g, self.vocab_size)
        return self.cache[key]


class _Compiled:
    def __init__(self, xgr, g, v):
        self.xgr, self.g, self.v = xgr, g, v

    def new_matcher(self):
        return _Matcher(self.xgr, self.xgr.GrammarMatcher(self.g), self.v)


class _Matcher:
    def __init__(self, xgr, m, v):
        self.xgr, self.m, self.v = xgr, m, v
        self.bm = xgr.allocate_token_bitmask(1, v)

    def bitmask(self):
        """The packed words of the allowed next tokens (no unpack)."""
        self.m.fill_next_token_bitmask(self.bm, 0)
        return self.bm[0][:(self.v + 31) // 32]

    def fill_bitmask(self, buf, row):
        """The packed words of the allowed next tokens into row `row` of buf (int32 [rows, >= ceil(vocab / 32)])."""
        self.m.fill_next_token_bitmask(buf, row)

    def mask(self):
        return unpack(self.bitmask(), self.v)

    def accept(self, tok):
        return self.m.accept_token(tok)

    def done(self):
        return self.m.is_terminated()


def unpack(words, v):
    """grammar.py:44-45: packed int32 words -> bool [v]."""
    w = torch.as_tensor(words, dtype=torch.int32)
    bits = (w[:, None] >> torch.arange(32, dtype=torch.int32)) & 1
    return bits.reshape(-1)[:v].bool()


def pack(mask):
    """bool [v] -> packed int32 words [ceil(v / 32)] (host helper; sample() packs bool masks on the GPU itself)."""
    m = np.asarray(mask.cpu() if isinstance(mask, torch.Tensor) else mask).astype(bool)
    n = (m.shape[0] + 31) // 32
    b = np.zeros(n * 32, dtype=np.uint64)
    b[:m.shape[0]] = m
    return torch.from_numpy((b.reshape(n, 32) << np.arange(32, dtype=np.uint64)).sum(1).astype(np.uint32)
                            .view(np.int32))


class MaskBatch:
    """The packed grammar masks of one step's rows (engine.py:272-273, :280 compute mask() per row and unpack it to
    bool [V]): matchers write their rows' words in place into one host buffer, int32 [rows, ceil(vocab / 32)], pinned
    when a GPU is present, and sample(..., masks=batch) sends the whole buffer to the device in one asynchronous copy
    on the launch stream. Rows that were not filled since the last reset() carry no mask. A batch may hold more rows
    than a call samples (one buffer sized for the largest batch): a call over n rows uses its first n.

    The copy reads the host buffer after sample() has been called, so refill it only once that call's results have
    been read (sample() returns them synchronously; after sample_ex, synchronize first)."""

    is_mask_batch = True

    def __init__(self, rows, vocab, pin=None):
        if rows <= 0 or vocab <= 0:
            raise ValueError(f"rows {rows} and vocab {vocab} must be > 0")
        self.rows, self.vocab, self.words = int(rows), int(vocab), (int(vocab) + 31) // 32
        pin = torch.cuda.is_available() if pin is None else bool(pin)
        self.host = torch.empty((self.rows, self.words), dtype=torch.int32, pin_memory=pin)
        self.filled = np.zeros(self.rows, dtype=bool)
        self._dev = None

    def reset(self):
        """Every row without a mask again (the words are left as they are and overwritten by the next fills)."""
        self.filled[:] = False

    def fill(self, row, matcher):
        """Row `row` from a matcher's fill_bitmask(buf, row) (xgrammar's fill_next_token_bitmask(bitmask, index))."""
        matcher.fill_bitmask(self.host, row)
        self.filled[row] = True

    def set(self, row, mask):
        """Row `row` from a bool [vocab] mask or packed int32 words [>= ceil(vocab / 32)]."""
        m = mask if isinstance(mask, torch.Tensor) else torch.from_numpy(np.asarray(mask))
        if m.dtype in (torch.int32, torch.uint32) and self.words <= m.numel() < self.vocab:
            w = m.reshape(-1)[:self.words]
            self.host[row].copy_(w.view(torch.int32) if w.dtype == torch.uint32 else w)
        elif m.numel() == self.vocab:
            self.host[row].copy_(pack(m.reshape(-1).to(torch.bool)))
        else:
            raise ValueError(f"mask of row {row} has {m.numel()} entries, the row has {self.vocab} tokens")
        self.filled[row] = True

    def device_words(self, dev, n=None):
        """The first n rows (all by default) of the buffer on `dev`: one copy from the host buffer, on the current
        stream of dev."""
        n = self.rows if n is None else int(n)
        if self._dev is None or self._dev.device != dev:
            self._dev = torch.empty((self.rows, self.words), dtype=torch.int32, device=dev)
        self._dev[:n].copy_(self.host[:n], non_blocking=True)
        return self._dev[:n]
