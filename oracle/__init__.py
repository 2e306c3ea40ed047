"""CPU oracle for the sigmoid-tension hot path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, never by the ``bozo_amd``
package.  ``tension_oracle`` is the float64 numpy restatement;
``torch_ref`` is the torch-on-CPU unfold restatement used as the CPU baseline
and as a second, independent formulation that pins the first.
"""
