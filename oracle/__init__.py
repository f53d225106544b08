"""CPU oracle for the neighborhood-attention path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference
natten-mlx ``pure`` backend and its helpers so the HIP library can be checked
against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
(``natten-mlx_amd/natten_amd``) never does and has no CPU fallback.

Modules and the reference code each follows:

* ``oracle.window`` — window start/end/pb_start (``utils/window.py:8-103``),
  the dilation-partition twin (``extras/allin1/reference_impl.py:13-45``),
  query positions and neighbor tables (``_core/pure.py:19-152``).
* ``oracle.na`` — fused/split forward, LSE, GQA, additional tokens +
  ``merge_attentions``, varlen, FMHA and the allin1 1D QK+RPB / AV
  (``_core/pure.py:155-808``, ``functional.py:29-828``, ``merge.py:20-68``,
  ``extras/allin1/__init__.py:40-109``, ``extras/allin1/functional.py:260-368``);
  backward is torch autograd of the float64 forward.
* ``oracle.brute`` — independent scalar loops for tiny inputs.

Pinning (what fixes each function beyond its own formula) is listed in each
module header; every function is pinned by at least one check in
``tests/test_oracle_*.py``.
"""
