"""Loader of oracle/_ref: the reference's own CPU sources compiled by oracle/Makefile (test infrastructure only).

    cpu()  -> module with adam_scalars, cpu_adam, cpu_gather, ... of srm2/csrc/srm2_cpu.cpp
    dir()  -> module with elara_dir_a / elara_dir_b of srm2/csrc/elara_dir.cpp (ATen; runs on CPU tensors)

Both return None when the build is absent (e.g. a checkout built without /root/reference).
"""
import glob
import importlib.util
from pathlib import Path

HERE = Path(__file__).resolve().parent / '_ref'
_mods = {}


def _load(name):
    if name not in _mods:
        hits = glob.glob(str(HERE / f'{name}*.so'))
        if not hits:
            _mods[name] = None
        else:
            import torch  # noqa: F401  (the extension links libtorch)
            spec = importlib.util.spec_from_file_location(name, hits[0])
            m = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(m)
            _mods[name] = m
    return _mods[name]


def cpu():
    return _load('elara_ref_cpu')


def dir():  # noqa: A001  (mirrors the reference's dir_ext())
    return _load('elara_ref_dir')
