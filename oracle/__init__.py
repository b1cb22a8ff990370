"""CPU oracle for the MXFP4 operator surface (test infrastructure only).

This package is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped operators live in ``mxfp4-gfx936_amd/mxfp4_amd`` and
fail loudly when their HIP library is missing; they never call into this
package.

Contents
--------
``mxfp4_oracle``  numpy / torch-CPU restatement of the reference algorithm
                  (explicit dequant, safe linear, safe routed MoE, the vLLM MoE
                  layer, routing metadata, both MXFP4 quantizers) plus FP64
                  accumulated oracles.
``c_oracle``      ctypes binding of ``mxfp4_oracle.c``: an independent integer
                  bit-construction of the same byte-level functions, used to
                  cross-check the numpy restatement and to check the kernels at
                  full sizes quickly.
"""
