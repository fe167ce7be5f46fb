"""Drop-in for goethe_engine/grammar.py: the same compiler / matcher surface, with the mask kept in xgrammar's packed
int32 form (token t allowed iff bit t % 32 of word t // 32 is set, LSB first; grammar.py:42-45) so that gse_sample
applies it on the GPU inside the fused pass instead of a host bool[V] unpack per row.

Matcher: mask() -> bool tensor [vocab] (as the reference); bitmask() -> int32 tensor [ceil(vocab / 32)] (packed, what
sample() consumes without unpacking); accept(tok) -> bool; done() -> bool.
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
