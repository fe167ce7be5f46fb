"""CPU oracle for the token-selection path (test infrastructure, not product code).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only as the checker or
as the timed CPU baseline. The product path (goethe-engine_amd) never imports it.

Modules:
  sampling_ref  numpy restatement of goethe_engine/sampling.py (+ the penalty / min-p / logprob extensions)
  spec_ref      numpy restatement of goethe_engine/spec.py mss and the tree-verify walk of engine.py _post
  cref          ctypes loader for the C restatement in oracle/c (splitmix64, greedy masked argmax, bit unpack)
"""
