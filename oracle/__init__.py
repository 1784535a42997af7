"""CPU oracle for the AttnRes routing path — test infrastructure only.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, as the checker or the timed CPU baseline.  The product
package ``kotodama_amd`` never imports it and has no CPU fallback.

``attnres_oracle``  float64 numpy restatement of the reference math and schedule
``torch_cpu_path``  the reference's CPU op sequence in torch (cpu baseline)

There is no ``oracle/_ref``: the reference path is Python/Triton, not C or
C++, so there is nothing of it to compile here.
"""
