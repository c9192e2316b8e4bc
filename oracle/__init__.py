"""CPU oracle of the ELARA sparse-update path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may import this package, and only as
the checker or the CPU baseline.  The product (elara_amd) never imports it and has no CPU fallback.

Contents
  elara_oracle.c  plain-C restatement, built into liboracle.so by oracle/Makefile (-O3 -ffp-contract=off)
  oracle.py       ctypes/numpy wrappers of liboracle.so
  ref.py          loader of oracle/_ref: the reference's own srm2_cpu.cpp and elara_dir.cpp compiled with g++
                  against this image's PyTorch (built only where /root/reference exists; the .so files travel)

How each function is pinned (checked against something other than itself; tests named in brackets)
  orc_adam_scalars   == reference adam_scalars from oracle/_ref for steps 0..10^4 and several hyperparameters;
                     closed forms bc1(1) = f32(1-b1), row 0 of the table zero      [tests/test_oracle.py]
  orc_cpu_adam       == reference cpu_adam from oracle/_ref, bitwise, on random states incl. duplicates across
                     steps and thread counts 1..16; == Triton golden vectors of srm2/ops.py _adam_rows
                     (tests/golden/triton_vectors.npz); invariants: untouched rows unchanged, first step from
                     m=v=0 gives m = omb1*g, v = (omb2*g)*g                                 [tests/test_oracle.py]
  orc_fmix32         MurmurHash3 published vectors (x86_32 of the empty key: seed 1 -> 0x514E28B7,
                     seed 0xFFFFFFFF -> 0x81F16F39, seed 0 -> 0); bijectivity via its inverse  [tests/test_oracle.py]
  orc_init_rows      == Triton golden vectors of srm2/gpu_ops.py _init_rows (ids >= 2^32, u32 wrap of r*D+j,
                     seeds >= 2^31, D not a power of two); range [-bound, bound), w0(0,0,seed 0) = -bound
  orc_replay_rows    == Triton golden vectors of srm2/gpu_ops.py _replay; == init + eager reference cpu_adam
                     (oracle/_ref) at the logged steps (test_replay.py:22-33 as an assertion)
  orc_segment_sum    == ATen's embedding_dense_backward (the op srm2/train.py:429 calls) run on the GPU, bitwise, on
                     both of its paths: <= 3072 indices (windows of 16) and the sorted path (runs of 10 from zero),
                     hot ids, all -0.0 ids (tests/golden/aten_segsum.npz, made by make_aten_segsum.py); properties
                     of both orders that other window or run lengths fail; torch.unique ordering and inverse;
                     column totals  [tests/test_dedup.py, tests/test_oracle.py]
  orc_dir_a/b        == reference elara_dir_a/elara_dir_b from oracle/_ref run on CPU tensors, whole directory
                     state and every output compared, over 60-step planner simulations in 5 configurations
                     (tests/dirsim.py); a hand-worked allocation sequence; invariants of srm2/train.py:474-477
                     (live == #valid entries, live + n_lfree == log_top)  [tests/test_directory.py]
                     In the Triton path's order (rel_cnt / rel arguments, srm2/elara_kernels.py): == the
                     reference's ELARAPlanner with dir_impl='triton' (its kernels in Triton's CPU interpreter),
                     per step and final state, 5 configurations (tests/golden/planner_vectors.npz); a hand-worked
                     step in both orders; equal to the default order in every state but the log ids
                     [tests/test_planner_golden.py, tests/test_directory.py]
"""
