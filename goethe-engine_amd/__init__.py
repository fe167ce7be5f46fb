"""goethe-engine_amd: goethe-engine's per-step token-selection path (sampling.py / grammar.py / spec.mss call surface)
on MI355X, with the arithmetic in hand-written HIP kernels for gfx950 (libgse.so, C ABI in include/gse.h).

The directory name holds a hyphen, so import it with importlib:

    import importlib
    ge = importlib.import_module("goethe-engine_amd")
    ge.sampling.sample(logits, params, seeds, idxs, masks)

Importing registers the alias "goethe_engine_amd" in sys.modules, after which `from goethe_engine_amd import sampling`
works too.
"""
import sys

from . import _lib, grammar, sampling, spec, workloads  # noqa: F401

sys.modules.setdefault("goethe_engine_amd", sys.modules[__name__])
