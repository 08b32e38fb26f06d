"""CPU oracle for the selective-SSM path -- TEST INFRASTRUCTURE ONLY.

This package is test infrastructure, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  Nothing under ``triton-ssm_amd/`` imports it, and the product path
has no CPU fallback: when the HIP library is missing it raises.

Contents
--------
``ssm_oracle``  float64 numpy restatement of every reference function on the
                path (each function cites the reference file:line it follows).
``oracle_c.c``  a plain-C fp32 restatement of the scan recurrences (OpenMP over
                independent rows), used as the timed CPU baseline ("port") and
                cross-checked against ``ssm_oracle`` by the CPU tests.
``cport``       ctypes loader for the built ``liboracle_c.so``.

How each function is pinned (i.e. checked against something other than a
retyping of its own formula) is listed in the header of ``ssm_oracle``.
"""
