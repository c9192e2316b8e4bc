"""elara_amd: MI355X-native (gfx950) sparse-update path of ELARA.

Hand-written HIP kernels behind a C-ABI (include/elara_amd.h, libelara_amd.so), exposed with the reference's op
signatures:
  elara_amd.ops        gpu_adam, ext().adam_scalars                       (srm2/ops.py)
  elara_amd.gpu_ops    init_rows, replay_rows, ScalarTable                 (srm2/gpu_ops.py)
"""
__version__ = '0.1.0'
