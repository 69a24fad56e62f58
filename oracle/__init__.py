"""CPU oracle for the packed FP8 top-8 MoE step.

TEST INFRASTRUCTURE ONLY. Nothing in the product package may import, call or
execute anything under ``oracle/``; only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker
(or as the timed CPU baseline), never as the thing that is measured or shipped.

The oracle restates, in numpy, the algorithm of the reference's hot path
(david6666666/drama-3-single-b300-inference, ``src/drama3``); each function
cites the reference file:line it follows.  Every function is pinned by a CPU
test in ``tests/test_oracle_*.py`` against a library routine (torch's
``float8_e4m3fn`` cast, ``torch.topk``, ``numpy.argsort(stable)``), a brute
force evaluation on tiny inputs, a closed form, or a known-answer trace taken
from the reference's own validators.  Functions whose reference lives in an
absent third-party dependency say "parity unpinned" in their docstring.
"""
