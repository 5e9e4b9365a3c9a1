"""CPU oracle for the quantized-MoE hot path -- TEST INFRASTRUCTURE ONLY.

This package is a NumPy restatement of the reference CPU path of raon-npu
(whguswka/raon-npu) for the q4nx mixture-of-experts hot path.  It exists so that
tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
can check the HIP implementation against the reference algorithm.  Product code
(``raon-npu_amd/``) never imports it: the product path fails loudly when its HIP
library is missing instead of falling back to anything here.

Modules and the reference files they restate (paths inside the reference tree):

* ``oracle.bf16``    -- ``quant/q4nx.py:32-124``, ``host/weights.py:104-123``
* ``oracle.q4nx``    -- ``quant/q4nx.py:127-438``, ``kernels/gemv/reference.py:34-79``
* ``oracle.moe``     -- ``host/backend.py:47-62,402-417,466-510``,
                        ``host/raon.py:1224-1247,1288-1330,1565-1621``,
                        ``kernels/moe/reference.py:127-180``
* ``oracle.planner`` -- ``kernels/moe_grouped/planner.py:18-322``

How each function is pinned (known answers, golden hashes, closed forms) is
listed in each module's docstring; functions whose parity is not pinned by any
check say "parity unpinned" there.
"""
