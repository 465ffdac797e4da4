"""CPU oracle for the in-context sparse attention hot path (test infrastructure only).

This package is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it.  The HIP backend under
``lightning-unified-video-editor-via-in-context-sparse-attention_amd/`` never imports it and
fails loudly when its native library is missing.

Modules
-------
``icsa_oracle``  vectorised PyTorch-CPU restatement of the reference path (fp64 by default,
                 fp32 for the CPU baseline), with optional injection of upstream decisions.
``bruteforce``   scalar numpy loops for tiny shapes; pins ``icsa_oracle`` independently.

Pinning status of every oracle function (which check pins it) is listed in the header of
``icsa_oracle``.
"""
from .icsa_oracle import *  # noqa: F401,F403
