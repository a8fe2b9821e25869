"""In-tree build of the gfx950 libraries (hipcc, no CUDA, no JIT cache).

libd1hip.so          environment, wait workload, LOS compiler, MFMA trunk layer, sampling, GAE, PPO step
libd1learn_clump0.so the d1-stairs-v2 learning task (learn_* ABI), CLUMP_MODE 0
libd1learn_clump1.so the same task with clumped placement in a third of resets
"""
import pathlib
import subprocess

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / 'csrc'
FLAGS = ['--offload-arch=gfx950', '-O3', '-std=c++17', '-fPIC', '-shared', '-ffp-contract=off',
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops']
TARGETS = {
    'libd1hip.so': ([CSRC / 'd1_env.hip', CSRC / 'd1_policy.hip', CSRC / 'd1_forward.hip', CSRC / 'd1_ppo.hip',
                     CSRC / 'd1_maps.hip'], []),
    'libd1learn_clump0.so': ([CSRC / 'd1_learn.hip'], ['-DD1_CLUMP_MODE=0']),
    'libd1learn_clump1.so': ([CSRC / 'd1_learn.hip'], ['-DD1_CLUMP_MODE=1']),
}


def build(verbose=False):
    jobs = []
    for name, (sources, defs) in TARGETS.items():
        out = HERE / name
        tmp = out.with_suffix('.so.tmp')
        cmd = ['hipcc', *FLAGS, *defs, '-I', str(HERE.parent / 'include'), '-o', str(tmp), *map(str, sources)]
        jobs.append((out, tmp, cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    errors = []
    for out, tmp, cmd, proc in jobs:
        _, err = proc.communicate()
        if proc.returncode:
            errors.append(f'{out.name}: hipcc failed:\n{err}')
            continue
        tmp.replace(out)
        if verbose:
            print(' '.join(cmd))
    if errors:
        raise RuntimeError('\n'.join(errors))
    return [out for out, *_ in jobs]


if __name__ == '__main__':
    print(build(verbose=True))
