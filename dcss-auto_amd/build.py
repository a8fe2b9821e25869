"""In-tree build of libd1hip.so for gfx950 (hipcc, no CUDA, no JIT cache)."""
import pathlib
import subprocess

HERE = pathlib.Path(__file__).resolve().parent
SOURCES = [HERE / 'csrc' / 'd1_env.hip', HERE / 'csrc' / 'd1_policy.hip']
FLAGS = ['--offload-arch=gfx950', '-O3', '-std=c++17', '-fPIC', '-shared', '-ffp-contract=off',
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops']


def build(verbose=False):
    out = HERE / 'libd1hip.so'
    tmp = out.with_suffix('.so.tmp')
    cmd = ['hipcc', *FLAGS, '-I', str(HERE.parent / 'include'), '-o', str(tmp), *map(str, SOURCES)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f'hipcc failed:\n{r.stderr}')
    tmp.replace(out)
    if verbose:
        print(' '.join(cmd))
    return out


if __name__ == '__main__':
    print(build(verbose=True))
