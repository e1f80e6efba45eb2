"""CPU oracle for the bytes_amd decode-attention hot path.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU, the semantics
of the saifmb0/bytes functions that bytes_amd replaces.  It is imported only
by ``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg
of ``bench.py``, and there only as the checker.  The product package
(``bytes_amd``) never imports, links or calls anything in here.

Pinning status of every function is listed in the module docstrings of
``oracle/reference.py`` ("Pinned by:") and checked in ``tests/test_oracle.py``.
"""
from . import reference  # noqa: F401
