"""Build recipe of libelara_amd.so (hipcc, gfx950 only).

Every .hip file under csrc/ is compiled on its own (in parallel) and linked into one shared library next to this
file.  Float flags: no FMA contraction, correctly rounded fp32 division and square root, denormals kept -- the
conditions under which the kernels are bitwise equal to the reference's CPU Adam.  Packed-fp32 instructions are
disabled for device code.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / 'csrc'
LIB = HERE / 'libelara_amd.so'
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
ARCH = 'gfx950'

CFLAGS = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}', '-ffp-contract=off', '-fno-fast-math',
          '-fhip-fp32-correctly-rounded-divide-sqrt', '-fno-gpu-flush-denormals-to-zero',
          '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
          '-Wall', '-Wno-unused-command-line-argument', f'-I{HERE.parent / "include"}']


def sources():
    return sorted(CSRC.glob('*.hip'))


def source_hash():
    """16 hex digits identifying the library's kernel code: SHA-256 over the compile flags, the C header and every
    kernel source and device header (by name and contents).  Profile summaries record it, so that a figure measured
    on other kernels can be recognised as stale."""
    import hashlib
    h = hashlib.sha256(' '.join(CFLAGS[:-1]).encode())
    for f in [HERE.parent / 'include' / 'elara_amd.h', *sorted(CSRC.glob('*.hip')), *sorted(CSRC.glob('*.h'))]:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def _compile(src, obj):
    cmd = [HIPCC, *CFLAGS, '-c', str(src), '-o', str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src.name}:\n{" ".join(cmd)}\n{r.stdout}\n{r.stderr}')
    return obj


def build(verbose=False):
    """Compile every kernel source and link libelara_amd.so (always rebuilds)."""
    objdir = HERE / '_build'
    objdir.mkdir(exist_ok=True)
    srcs = sources()
    objs = [objdir / (s.stem + '.o') for s in srcs]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(_compile, srcs, objs))
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [HIPCC, '-shared', f'--offload-arch={ARCH}', '-o', str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'link failed:\n{" ".join(cmd)}\n{r.stdout}\n{r.stderr}')
    os.replace(tmp, LIB)
    if verbose:
        print(f'built {LIB}', file=sys.stderr)
    return LIB


if __name__ == '__main__':
    build(verbose=True)
