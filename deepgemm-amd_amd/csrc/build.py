"""Build libdeepgemm_mi355x.so for gfx950 in-tree.

Device sources (*.hip) are compiled by hipcc for --offload-arch=gfx950; the
host API (*.cpp) is plain C++ compiled by g++ against the HIP runtime headers.
All objects are linked by hipcc into deep_gemm/libdeepgemm_mi355x.so next to the
Python package, so the library travels with the source tree.

Usage: python deepgemm-amd_amd/csrc/build.py [--jobs N] [--verbose]
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, 'include')
OBJ_DIR = os.path.join(PKG, '_build')
LIB_PATH = os.path.join(PKG, 'deep_gemm', 'libdeepgemm_mi355x.so')
ROCM = os.environ.get('ROCM_PATH', '/opt/rocm')
HIPCC = os.path.join(ROCM, 'bin', 'hipcc')

ARCH = 'gfx950'
COMMON = ['-O3', '-std=c++20', '-fPIC', '-Wall', '-I', INCLUDE, '-I', HERE]
# Packed FP32 VALU ops are disabled for every device compile.
# MFMA results are kept in architectural VGPRs (the promotion FMAs read them
# directly; AGPR destinations would cost a v_accvgpr_read per element).
HIP_FLAGS = ['--offload-arch=' + ARCH, '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
             '-ffp-contract=fast-honor-pragmas', '-mllvm', '-amdgpu-mfma-vgpr-form=true',
             # the LDS-DMA asm helpers clobber M0, which no compiled code here keeps live
             '-Wno-inline-asm']
CXX_FLAGS = ['-D__HIP_PLATFORM_AMD__', '-I', os.path.join(ROCM, 'include')]


def sources():
    out = []
    for name in sorted(os.listdir(HERE)):
        if name.endswith('.hip') or name.endswith('.cpp'):
            out.append(os.path.join(HERE, name))
    return out


def _compile(src, verbose):
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + '.o')
    if src.endswith('.hip'):
        cmd = [HIPCC] + COMMON + HIP_FLAGS + ['-c', src, '-o', obj]
    else:
        cmd = ['g++'] + COMMON + CXX_FLAGS + ['-c', src, '-o', obj]
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise.
    err = '\n'.join(l for l in res.stderr.splitlines() if 'packed-fp32-ops' not in l)
    if res.returncode != 0:
        raise RuntimeError(f'compile failed: {src}\n{err}')
    if verbose and err.strip():
        print(err, flush=True)
    return obj


def build(jobs=None, verbose=False):
    if not os.path.exists(HIPCC):
        raise RuntimeError(f'hipcc not found at {HIPCC}')
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_PATH + '.tmp'
    cmd = [HIPCC, '--offload-arch=' + ARCH, '-shared', '-fPIC', '-o', tmp] + objs
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError('link failed:\n' + res.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def clean():
    shutil.rmtree(OBJ_DIR, ignore_errors=True)
    if os.path.exists(LIB_PATH):
        os.remove(LIB_PATH)


if __name__ == '__main__':
    ap = argparse.ArgumentParser()
    ap.add_argument('--jobs', type=int, default=None)
    ap.add_argument('--verbose', action='store_true')
    ap.add_argument('--clean', action='store_true')
    args = ap.parse_args()
    if args.clean:
        clean()
    print(build(args.jobs, args.verbose))
    sys.exit(0)
