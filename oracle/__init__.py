"""CPU restatement of ditserve's per-step DiT forward — TEST INFRASTRUCTURE ONLY.

This package is the oracle: a plain PyTorch-CPU (fp32, optionally fp64)
restatement of the arithmetic the reference runs for one Wan2.1/Wan2.2 DiT
block, the Wan packet prelude/epilogue, and the SD3.5 packed MMDiT joint block.
Each function cites the reference file:line it follows (paths relative to the
reference repository root).

The functions run wherever their inputs live: on the CPU as the restatement
proper, and (a GPU test's full-size check only) on a GPU device in fp32, where the
same torch operations compute the same formulas.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline.  The product (``ditserve_amd``) never imports it: the GPU path fails
loudly when its HIP library is missing instead of falling back to this code.

Pinning status (what checks each function against something it does not
restate; see ``tests/test_oracle_pinning.py``):
  * packing.build_cu_seqlens / packing_stats / packed_plan: reference golden
    vectors from tests/python/test_domain_block_executor.py:689-698,769,915-916.
  * common.layer_norm / rms_norm / gelu_tanh / timestep_embedding / sdpa:
    float64 closed forms and torch.nn.functional library routines.
  * wan.rope_freqs / apply_rotary: norm preservation, identity at position 0,
    relative-position property of q.k, and the closed-form angle table.
  * wan.block_forward / sd35.joint_block_forward: composition of the pinned
    pieces; packed == per-segment by construction.  The exact op order and
    casts inside diffusers 0.36.0 (not present in the reference tree, not
    installable offline) are "parity unpinned" beyond the in-tree restatements
    at workers/ditserve/models/wan/block.py:276-297 and
    workers/ditserve/models/sd35_batch.py:336-736.
"""
