"""CPU oracle for the GGUF dequant + quantized matvec path.

TEST INFRASTRUCTURE ONLY. Nothing in the shipped package (``flatrun_amd``)
imports this package. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import, call or link anything under
``oracle/``, and only to check results or as the CPU baseline, never as the
thing measured or shipped.

Contents
--------
``gguf_np``     NumPy restatement of the reference dequantizers
                (``src/flatrun/dequant/gguf.py``), same op order and dtypes,
                plus the NumPy reference matvec (``runtime/backend.py:203-213``)
                and an fp64 matvec used as the accuracy yardstick.
``native_ref.c``  C restatement of the reference's scalar native kernels
                (``src/flatrun_native/kernels/q4_k.h``, ``q6_k.h``,
                ``q8_0.h``) with x86 semantics (no FMA contraction, single
                thread, same accumulation order), built into
                ``oracle/liboracle.so`` by ``oracle/Makefile``.
``_ref/``       The reference's own ``_C`` module compiled from its sources
                under /root/reference (see ``oracle/Makefile``); git-ignored,
                absent on machines without the reference checkout.
``loader``      ctypes / importlib loaders for the two native builds above.

Parity pins (what each oracle function is checked against) are listed in the
header of each module and exercised in ``tests/test_oracle_*.py``.
"""
