"""ctypes binding of libelara_amd.so (the C-ABI declared in include/elara_amd.h).

PyTorch supplies device memory and streams; the kernels are the library's.  There is no fallback: if the
library is missing, every op raises.  torch is imported before the library is loaded so that the library binds
to the HIP runtime torch already loaded (same soname), and torch's streams are valid handles for it.
"""
import contextlib
import ctypes
import os
import threading
from pathlib import Path

import torch

# ELARA_AMD_LIB may name another build of the same library (e.g. a tuning variant); default: the in-tree build.
LIB_PATH = Path(os.environ.get('ELARA_AMD_LIB') or (Path(__file__).resolve().parent / 'libelara_amd.so'))

_lib = None
_lock = threading.Lock()

c_i64, c_i32, c_u32, c_f32, c_f64, c_vp = (ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float,
                                           ctypes.c_double, ctypes.c_void_p)
c_f32p = ctypes.POINTER(ctypes.c_float)

# name -> (restype, argtypes); must match include/elara_amd.h
SIGNATURES = {
    'elr_error_string': (ctypes.c_char_p, [ctypes.c_int]),
    'elr_version': (ctypes.c_int, []),
    'elr_host_device_ptr': (ctypes.c_int, [c_vp, ctypes.POINTER(c_vp)]),
    'elr_adam_scalars': (None, [c_f64, c_f64, c_f64, c_f64, c_i64, c_f32p]),
    'elr_cpu_adam': (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_f32p, ctypes.c_int]),
    'elr_scalar_table': (ctypes.c_int, [c_f64, c_f64, c_f64, c_f64, c_i64, c_vp]),
    'elr_adam_rows': (ctypes.c_int, [c_vp, c_i64, c_vp, ctypes.c_int, c_vp, c_i64, c_i64, c_f32p, c_vp]),
    'elr_adam_rows_timed': (ctypes.c_int, [c_vp, c_i64, c_vp, ctypes.c_int, c_vp, c_i64, c_i64, c_f32p, c_vp, c_vp,
                                           c_vp]),
    'elr_init_rows': (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_u32, c_f32, c_vp]),
    'elr_scalar_recip': (ctypes.c_int, [c_vp, c_i64, c_vp]),
    'elr_replay_rows': (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_int, c_u32,
                                       c_f32, c_vp, c_vp, c_i64, c_vp]),
    'elr_replay_rows_timed': (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_int,
                                             c_u32, c_f32, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp]),
    'elr_dir_scratch_bytes': (c_i64, [c_i64, c_i64]),
    'elr_dedup_scratch_bytes': (c_i64, [c_i64, c_i64]),
    'elr_selfcheck_div': (ctypes.c_int, [c_f32, c_vp, c_vp, c_vp]),
    'elr_selfcheck_sqrt': (ctypes.c_int, [c_vp, c_vp, c_vp]),
    'elr_selfcheck_quot': (ctypes.c_int, [c_f32, c_vp, c_vp, c_vp, c_vp]),
    'elr_copy_rows': (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    'elr_mark_rows': (ctypes.c_int, [c_vp, c_vp, c_i64, c_i32, c_vp, c_i64, c_vp, c_u32, c_vp]),
    'elr_glog_put': (ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp]),
    'elr_glog_take': (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp]),
    'elr_unique': (ctypes.c_int, [c_vp, c_i64, ctypes.c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp]),
    'elr_segment_sum': (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_vp]),
    'elr_adam_dedup': (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_f32p, c_vp, c_i64, c_vp]),
    'elr_adam_dedup_noalloc': (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_f32p, c_vp]),
    'elr_dir_a': (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64] + [c_vp] * 9
                  + [c_vp, c_i64, c_vp]),
    'elr_dir_evict': (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp]),
    'elr_dir_evict_deferred': (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                              c_i64, c_vp]),
    'elr_dir_a_deferred': (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64] + [c_vp] * 10
                           + [c_vp, c_i64, c_vp]),
    'elr_dir_b_release': (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, ctypes.c_int, c_vp, c_vp,
                                         c_i64, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp]),
    'elr_dir_b': (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_i64,
                                 c_vp]),
    'elr_plan_scratch_bytes': (c_i64, [c_i64, c_i64]),
    'elr_plan_admit': (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, ctypes.c_int, c_i64, c_i64, c_i64, c_i64, ctypes.c_int,
                                      c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    'elr_plan_admit_slots': (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, ctypes.c_int, c_i64, c_i64, c_i64, c_i64,
                                            ctypes.c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    'elr_assemble': (ctypes.c_int, [c_vp, c_vp]),
    'elr_step_exec_bytes': (c_i64, [c_vp]),
    'elr_step_exec': (ctypes.c_int, [c_vp, c_vp, c_i64, c_vp, c_vp]),
    'elr_abi_sizes': (ctypes.c_int, [c_vp, ctypes.c_int]),
    'elr_step_update': (ctypes.c_int, [c_vp, c_vp]),
    'elr_dedup_plan_bytes': (c_i64, [c_i64, c_i64]),
    'elr_dedup_plan': (ctypes.c_int, [c_vp, c_i64, ctypes.c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp]),
    'elr_dedup_plan_fields': (ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, ctypes.c_int, c_vp, c_vp, c_vp, c_vp, c_i64,
                                             c_i64, c_vp]),
    'elr_segment_sum_plan': (ctypes.c_int, [c_vp, c_i64, c_i64, ctypes.c_int, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp]),
    'elr_segment_sum_plan_final': (ctypes.c_int, [c_vp, c_i64, c_i64, ctypes.c_int, c_vp, c_i64, c_vp, c_vp, c_i64,
                                                  c_vp]),
    'elr_adam_dedup_plan': (ctypes.c_int, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, ctypes.c_int, c_vp, c_i64, c_vp,
                                           c_vp]),
    'elr_plan_classify': (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp]),
    'elr_plan_classify_seg': (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, ctypes.c_int, c_vp, c_i64,
                                             c_vp]),
    'elr_plan_step_scratch_bytes': (c_i64, [c_i64, c_i64]),
    'elr_plan_step': (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, ctypes.c_int, c_vp, c_i64,
                                     c_vp]),
    'elr_step_exec_dev_bytes': (c_i64, [c_vp]),
    'elr_step_exec_dev': (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp]),
    'elr_step_dev_bytes': (c_i64, [c_vp]),
    'elr_step_dev': (ctypes.c_int, [c_vp, c_vp, c_i64, c_vp, c_vp]),
}

DIR_FIELDS = ('code', 'loc', 'ent', 'lstep', 'lfree', 'n_lfree', 'log_top', 'mat_top', 'live', 'adm_c0', 'rj',
              'pstep', 'kthr', 'toff', 'slot_of', 'slot_row', 'rok')


class DirState(ctypes.Structure):
    """elr_dir_state: the 17 device pointers of the directory (srm2/csrc/elara_dir.cpp:8-10) and T."""
    _fields_ = [(n, c_vp) for n in DIR_FIELDS] + [('T', c_i64)]


class DirParams(ctypes.Structure):
    """elr_dir_params: the reference's pv = (R, K, Lcap, n0, Cdyn, MAT, trash, evl) (elara_dir.cpp:11)."""
    _fields_ = [(n, c_i64) for n in ('R', 'K', 'Lcap', 'n0', 'Cdyn', 'MAT', 'trash', 'evl')]


class PlanIn(ctypes.Structure):
    """elr_plan_in: inputs of the planner classification (srm2/elara.py:214-267)."""
    _fields_ = [('u', c_vp), ('n', c_i64), ('next', c_vp * 4), ('n_next', c_i64 * 4), ('nnext', ctypes.c_int),
                ('slot_of', c_vp), ('last_seen', c_vp), ('code', c_vp), ('kthr', c_vp), ('toff', c_vp), ('T', c_i64),
                ('dyn', c_vp), ('nd', c_i64), ('slot_row', c_vp), ('mat_top', c_vp), ('log_top', c_vp),
                ('s', c_i64), ('K', ctypes.c_int), ('want_t', ctypes.c_int), ('loc', c_vp), ('R', c_i64),
                ('next_bits', c_vp), ('next_mask', c_u32), ('carry', ctypes.c_int), ('live', c_vp), ('n_dev', c_vp),
                ('nd_dev', c_vp)]


# the device-driven step (elr_plan_step / elr_step_exec_dev): descriptor and control-state words
DESC_WORDS, CTL_WORDS = 40, 32
D_B, D_NEV, D_KEEP_OFF, D_NKEEP, D_NFREE, D_NADM, D_LAZY, D_NL = 0, 11, 12, 13, 14, 15, 16, 17
D_SKIP, D_OVERFLOW, D_TAKE, D_BARRIER, D_NROWS, D_ND, D_MAT_HI, D_LOG_HI = 28, 29, 30, 31, 32, 33, 34, 35
S_NFREE, S_ND, S_ERR, S_ERR_STEP, S_ERR_A, S_ERR_B, S_ERR_C, S_STATS = 0, 1, 2, 3, 4, 5, 6, 8
STEP_ERR_ROWS, STEP_ERR_CAPACITY = 1, 2
STAT_KEYS = ('hits', 'N', 'L', 'F', 'S', 'adm', 'ev', 'preempt', 'overflow', 'compactions', 'appends', 'barriers',
             'steps')


class PlanCtl(ctypes.Structure):
    """elr_plan_ctl: the device-driven step's control state, descriptor and capacity bounds."""
    _fields_ = [('state', c_vp), ('desc', c_vp), ('mat_cap', c_i64), ('log_cap', c_i64), ('triton', c_i64)]


class PlanOut(ctypes.Structure):
    """elr_plan_out: per-position classes, flags, slots and codes, the class order, the dynamic-slot partition and
    the host counts; optionally the rows, codes and slots in class-rank order and the L rows in reference order."""
    _fields_ = [('cls', c_vp), ('flags', c_vp), ('sl', c_vp), ('c', c_vp), ('order', c_vp), ('rank', c_vp),
                ('dyn_out', c_vp), ('counts', c_vp), ('u_ord', c_vp), ('c_ord', c_vp), ('sl_ord', c_vp),
                ('L_row', c_vp), ('L_cnt', c_vp), ('loc_ord', c_vp)]


class AssembleArgs(ctypes.Structure):
    """elr_assemble_args: the fused weight assembly of one step (srm2/elara.py:471-489)."""
    _fields_ = [('work', c_vp), ('rows', c_vp), ('n', c_i64), ('D', c_i64), ('K', ctypes.c_int),
                ('nseg', ctypes.c_int), ('seg_end', c_i64 * 16), ('seg_kind', ctypes.c_int * 16),
                ('seg_aux', c_i64 * 16), ('seed', c_u32), ('bound', c_f32), ('L_ids', c_vp), ('L_steps', c_vp),
                ('L_cnt', c_vp), ('nL', c_i64), ('logs', c_vp), ('nlogs', c_i64), ('table', c_vp), ('recip', c_vp),
                ('table_rows', c_i64), ('mat', c_vp), ('mat_rows', c_i64), ('loc', c_vp), ('R', c_i64)]



class SlotsArgs(ctypes.Structure):
    """elr_slots_args: the pool-slot bookkeeping of a step's admissions (srm2/elara.py:345-347, 368)."""
    _fields_ = [('free_stack', c_vp), ('n_free', c_i64), ('ev_slot', c_vp), ('nev', c_i64), ('keep', c_vp),
                ('nkeep', c_i64), ('adm_slots', c_vp), ('dyn_out', c_vp)]


class UpdateArgs(ctypes.Structure):
    """elr_update_args: the executor's update of one step (srm2/elara.py:491-580)."""
    _fields_ = [('D', c_i64), ('K', c_i64), ('pool', c_vp), ('pool_rows', c_i64), ('mat', c_vp), ('mat_rows', c_i64),
                ('logs', c_vp), ('log_rows', c_i64), ('glog', c_vp), ('glog_slots', c_i64), ('grad', c_vp),
                ('work', c_vp), ('b', c_i64 * 11), ('step', c_i64), ('lr', ctypes.c_double), ('b1', ctypes.c_double),
                ('b2', ctypes.c_double), ('eps', ctypes.c_double), ('evl', ctypes.c_int32), ('hit_slot', c_vp),
                ('hrec_dyn', c_vp), ('hrec_j', c_vp), ('nev', c_i64), ('ev_slot', c_vp), ('evf_slots', c_vp),
                ('evl_ids', c_vp), ('ev_dyn', c_vp), ('adm_slots', c_vp), ('lazy_n', c_i64), ('n0', c_i64),
                ('c_slots', c_vp), ('a_ids', c_vp), ('fn_slot', c_vp), ('s_slot', c_vp), ('part', ctypes.c_int32),
                ('link_blocks', c_i64)]


class ExecArgs(ctypes.Structure):
    """elr_exec_args: the rest of a planned step in one call (elr_step_exec)."""
    _fields_ = [('dir', DirState), ('pv', DirParams), ('s', c_i64), ('b', c_i64 * 11), ('u_ord', c_vp), ('c_ord', c_vp),
                ('sl_ord', c_vp), ('loc_ord', c_vp), ('L_row', c_vp), ('L_cnt', c_vp), ('slots', SlotsArgs),
                ('seed', c_u32), ('bound', c_f32), ('table', c_vp), ('recip', c_vp), ('table_rows', c_i64),
                ('upd', UpdateArgs), ('dir_order', c_i64), ('link_stream', c_vp), ('link_start', c_vp),
                ('link_done', c_vp), ('link_wait', c_vp)]


EXEC_OUT_FIELDS = ('L_steps', 'L_ids', 'hrec_dyn', 'hrec_j', 'ev_row', 'rep', 'evl_ids', 'evf_slots', 'ev_dyn',
                   'adm_slots', 'a_ids', 'c_slots', 'work')


class ExecOut(ctypes.Structure):
    """elr_exec_out: byte offsets in the workspace of the arrays elr_step_exec writes."""
    _fields_ = [(n, c_i64) for n in EXEC_OUT_FIELDS]


class StepDevArgs(ctypes.Structure):
    """elr_step_dev_args: a whole device-driven step in one call."""
    _fields_ = [('plan', PlanIn), ('ctl', PlanCtl), ('grad', c_vp), ('n_occ', c_i64), ('key_bits', c_i64),
                ('dplan', c_vp), ('dplan_bytes', c_i64), ('exec', ExecArgs), ('mark_rows', c_vp), ('mark_n', c_vp),
                ('mark_nmax', c_i64), ('mark_value', c_i64), ('mark_bit', c_i64), ('mark_event', c_vp)]


STEP_DEV_OUT_FIELDS = ('cls', 'flags', 'sl', 'c', 'order', 'rank', 'dyn_out', 'counts', 'u_ord', 'c_ord', 'sl_ord',
                       'L_row', 'L_cnt', 'loc_ord', 'grad_rows', 'exec_ws')


class StepDevOut(ctypes.Structure):
    """elr_step_dev_out: byte offsets in the step's workspace of the plan's outputs, G and the executor's arrays."""
    _fields_ = [(n, c_i64) for n in STEP_DEV_OUT_FIELDS] + [('exec', ExecOut)]


ABI_STRUCTS = (DirState, DirParams, PlanIn, PlanOut, AssembleArgs, SlotsArgs, UpdateArgs, ExecArgs, ExecOut, PlanCtl,
               StepDevArgs, StepDevOut)


def lib():
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(f'{LIB_PATH} is missing: build it with `python -c "import __graft_entry__ as g; '
                                       f'g.build()"` (no CPU fallback exists)')
                L = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    f = getattr(L, name)
                    f.restype = res
                    f.argtypes = args
                _lib = L
    return _lib


def check(rc, what):
    """Raise RuntimeError for a nonzero C-ABI return code (the reference raises through TORCH_CHECK)."""
    if rc != 0:
        msg = lib().elr_error_string(rc).decode()
        raise RuntimeError(f'{what} failed ({rc}): {msg}')


# torch's own C entry points for the current device and raw stream handle (what torch.cuda.current_stream reads,
# without building a Stream object: about 0.1 us against 2 us per call); the public API where they are absent.
_raw_stream = getattr(torch._C, '_cuda_getCurrentRawStream', None)
_cur_device = getattr(torch._C, '_cuda_getDevice', None)
_NO_SWITCH = contextlib.nullcontext()


def _index_of(dev):
    return dev.index if dev.index is not None else torch.cuda.current_device()


def stream_of(t):
    """Raw hipStream_t of torch's current stream on t's device."""
    return ctypes.c_void_p(raw_stream(t.device))


def raw_stream(dev):
    """torch's current stream on device `dev` as an integer handle."""
    if _raw_stream is not None:
        return _raw_stream(_index_of(dev))
    return torch.cuda.current_stream(dev).cuda_stream


def on_device(dev):
    """Context that makes `dev` the current HIP device for a launch (no switch when it already is)."""
    if _cur_device is not None and _cur_device() == _index_of(dev):
        return _NO_SWITCH
    return torch.cuda.device(dev)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def is_arena(t):
    """A float32 contiguous tensor the kernels can reach: in HBM, or in pinned host memory (the capacity tier)."""
    return t.dtype == torch.float32 and t.is_contiguous() and (t.is_cuda or (t.device.type == 'cpu' and t.is_pinned()))


def dptr(t):
    """Device-visible address of t's data: a GPU tensor's own address, or for a pinned host tensor the address HIP
    maps it to (elr_host_device_ptr; raises if the memory is not pinned and mapped)."""
    if t is None:
        return ctypes.c_void_p(0)
    if t.is_cuda:
        return ctypes.c_void_p(t.data_ptr())
    if t.device.type == 'cpu' and t.is_pinned():
        if t.numel() == 0:
            return ctypes.c_void_p(0)
        d = c_vp()
        check(lib().elr_host_device_ptr(ctypes.c_void_p(t.data_ptr()), ctypes.byref(d)), 'elr_host_device_ptr')
        return ctypes.c_void_p(d.value)
    raise RuntimeError('tensor must be on the GPU or in pinned host memory')


def scalars8(vals):
    return (ctypes.c_float * 8)(*vals)


def split_empty(dev, dtype, sizes):
    """Uninitialised 1-D tensors of the given sizes, views of one allocation: one allocator call and one split for a
    launch's outputs of one dtype (fewer Python-level tensor constructions than an allocation each)."""
    return torch.empty(sum(sizes), dtype=dtype, device=dev).split(list(sizes))


ESIZE = {torch.int8: 1, torch.bool: 1, torch.uint8: 1, torch.int32: 4, torch.int64: 8, torch.float32: 4}
