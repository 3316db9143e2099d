"""CPU oracle for the windowed-attention hot path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``atflash-kernel_amd/``) imports, links or runs this
package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may use it, and only as the checker (or, for the CPU
baseline, as the timed CPU restatement), never as the thing that is measured on
the GPU or shipped.

Modules
  window_rule  stdlib restatement of the window rule and its integer tables
               (reference: atflash/window_table.py, window_tables/atflash_window.py,
               kernels/flashinfer_port/fiwin_common.py:35-60,
               microbench/b1_correctness.py:40-58).
  attention    torch-CPU fp32/fp64 restatement of the banded reference attention
               (atflash/reference.py:27-80), the HF rotate-half RoPE
               (microbench/b1_correctness.py:113-135), the sliced decode oracle
               (gates/g2_correctness.py:37-76) and the log-sum-exp merge.

How each function is pinned (golden vectors, closed forms, brute force) is
listed in the module headers.  A function without such a check would be marked
"parity unpinned" there; at present every function has at least one pin.
"""
