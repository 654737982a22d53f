"""``import wmma_ops`` -- the reference's module name for this library.

The reference builds its PyTorch extension as the module ``wmma_ops`` (setup.py:18-21) and
its tests and callers ``import wmma_ops`` (test_rocwmma_patch.py:43,
test_fragment_loading.py:53).  Importing this module yields the ``wmma_ops_amd`` package
object itself (the same functions, the same HIP library), so code written against the
reference runs unchanged with this repository's root on ``sys.path``.
"""
import sys as _sys

import wmma_ops_amd as _impl

_sys.modules[__name__] = _impl
