"""The reference's low-level extension object (`src/pck/cuda/_ext.py`): ``extension()`` returns
the native entry points under the names the reference's pybind module exports
(`src/pck/cuda/csrc/bindings.cpp:302-335`), here bound to libpck_hip.so."""

from __future__ import annotations

import functools
from types import SimpleNamespace

from pck.cuda._lib import lib


@functools.cache
def extension() -> SimpleNamespace:
    from pck.cuda import gemv
    from pck.cuda.checker import blocked_check
    from pck.cuda.sampling import sampling_check
    from pck.cuda.template import _column, _template, _template_q8

    lib()  # fail here, loudly, if the library is not built
    return SimpleNamespace(
        gemv_naive=lambda W, x, threads: gemv.gemv_naive(W, x, threads),
        gemv_coalesced=lambda W, x, threads: gemv.gemv_coalesced(W, x, threads),
        gemv_fp8=lambda Q, x, threads: gemv.gemv_fp8(Q, x, threads),
        blocked_check=blocked_check,
        sampling_check=sampling_check,
        gemv_template=_template,
        gemv_template_q8=_template_q8,
        gemv_column=_column,
    )
