"""CPU fp32 oracle of the Token2Wav hot path (test infrastructure only).

This package restates, in plain PyTorch fp32 on the CPU, what the reference engine computes on the path that the
MI355X kernels replace: the DiT estimator inside the classifier-free-guided Euler CFM loop, its streaming key/value and
causal-conv state, and the HiFT vocoder with its streaming glue.  Every function cites the reference file and lines it
follows (paths relative to the reference repository root).

It is a checker, never the thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import it.  The product package never imports it and fails loudly when its HIP
library is missing.

Parity status per module is stated in each module's docstring.  Parts of the model that live inside the third-party
``stepaudio2`` package (``minicpmo-utils==1.0.6``: timestep embedder, adaLN internals, HiFT geometry, ...) are not
visible in the reference repository; the oracle defines them (CosyVoice2-style defaults) and they are "parity unpinned"
against the real stepaudio2 modules.
"""
