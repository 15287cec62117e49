"""CPU oracle of the cascade-decode operator set -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's cascade-decode
path so the HIP kernels can be checked against it. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it, and only as the checker. The product (``vllm-hust-cascade-kernel_amd/``)
never imports it and has no CPU fallback.

Modules and the reference code each follows (paths relative to the reference root):

* ``bf16``      -- round-to-nearest-even float32 -> bfloat16 (the ``bf16()`` helper of
                   ``ascend-kernel/csrc/ops/fa_fp32_stage1/test/fa_fp32_ref.py:25-27``).
* ``attention`` -- paged stage-1 attention with 512-column online softmax and bf16 P
                   (``fa_fp32_ref.py:68-245``), the padded LSE layout
                   (``.../block_epilogue_rescale_o_no_split_row.hpp:367-419``), the
                   per-sequence suffix attention and the full cascade.
* ``merge``     -- the LSE merge closed form (``ascend-kernel/csrc/ops/lse_merge/test/
                   lse_merge_cases.py:45-50``) and its fp32 operation order
                   (``.../op_kernel/kernel_lse_merge.cpp:237-289``).
* ``gemm``      -- gate_up GEMM with the f3 epilogue modes
                   (``ascend-kernel/csrc/ops/f3_floor/op_kernel/kernel_f3_floor.cpp:150-308``,
                   ``.../f3_floor/design.md:94-111``).
* ``inputs``    -- seeded input generators (``fa_fp32_ref.py:30-61``,
                   ``lse_merge_cases.py:32-42``) extended with permuted block tables.

Pinning. Each function is checked in ``tests/test_oracle_*.py`` against the
reference's fixtures (``tests/golden/``) and against what mathematics fixes
(dense softmax, closed forms, brute force on tiny inputs, library routines),
with planted-mistake tests showing those checks are sensitive. The suffix
attention is pinned only through the shared stage-1 arithmetic and dense
attention: the reference's real stage 2 (CANN FIA v2) is closed, so parity with
it is unpinned.
"""
