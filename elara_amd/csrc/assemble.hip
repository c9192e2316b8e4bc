// Fused weight assembly of one ELARA step (srm2/elara.py:471-489, ELARAExecutor.assemble): the full states of the
// non-resident rows the step touches, written into one work array in the planner's class-rank order, in a single
// launch.  Each work row belongs to a segment of one kind:
//   INIT    counter-hash initial state of an implicit (N) row                         (srm2/gpu_ops.py:26-48)
//   REPLAY  init plus exact replay of a logged (L) row's entries, read from the log arena by entry id
//                                                                                     (srm2/gpu_ops.py:51-79)
//   GATHER  the state of a materialised (M) row, read from the MAT arena at loc[row]
// The segments are ranges of work positions given by the caller; a replay segment names where its rows' entry ids,
// steps and counts start in the directory's replay inputs (elr_dir_a's steps / ids, in the caller's L-row order).
// Rows whose inputs are out of range are skipped (left unwritten), as elsewhere in this library.
// D = 64, 128, 256, 512 with 16-byte aligned arrays: a wave per row, each lane holding D/64 consecutive floats
// (elr_rowio.h).  Any other D or alignment: the generic kernel, a wave per row whose lanes step through the row one
// float at a time.  K <= 8.
#include "elr_asm_dev.h"

namespace elr {

int assemble_check(const elr_assemble_args& a) {
  if (a.n < 0 || a.nseg < 1 || a.nseg > ELR_ASM_MAX_SEG || a.K < 1 || a.D < 1) return ELR_EINVAL;
  if (a.K > 8) return ELR_EUNSUPPORTED;
  if (a.n == 0) return ELR_OK;
  if (a.n > (int64_t(1) << 31) - 4 || !a.work || !a.rows) return ELR_EINVAL;
  int64_t prev = 0;
  bool need_replay = false, need_gather = false;
  for (int g = 0; g < a.nseg; ++g) {
    if (a.seg_end[g] < prev || a.seg_kind[g] < ELR_ASM_INIT || a.seg_kind[g] > ELR_ASM_GATHER) return ELR_EINVAL;
    if (a.seg_end[g] > prev) {
      need_replay |= a.seg_kind[g] == ELR_ASM_REPLAY;
      need_gather |= a.seg_kind[g] == ELR_ASM_GATHER;
    }
    prev = a.seg_end[g];
  }
  if (prev != a.n) return ELR_EINVAL;
  if (need_replay && (!a.L_ids || !a.L_steps || !a.L_cnt || !a.logs || !a.table || !a.recip || a.nL < 0))
    return ELR_EINVAL;
  if (need_gather && (!a.mat || !a.loc)) return ELR_EINVAL;
  return ELR_OK;
}

}  // namespace elr

extern "C" int elr_assemble(const elr_assemble_args* args, void* stream) {
  using namespace elr;
  if (!args) return ELR_EINVAL;
  const elr_assemble_args& a = *args;
  const int rc = assemble_check(a);
  if (rc || a.n == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  assemble_visit(a, [&](const auto& f, int64_t blocks) { launch1(f, blocks, st); });
  return launch_status();
}
