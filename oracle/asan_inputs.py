"""TEST INFRASTRUCTURE ONLY — writes the raw inputs of oracle/asan_driver.c into a directory
(map 1057 floor and spawnable cells, the ray table, five env configurations, the learning
task's tables and configuration), so the sanitizer build runs as a plain executable: a
sanitized library loaded into Python would not see Python's allocations."""
import ctypes as C
import importlib
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
pkg = importlib.import_module('dcss-auto_amd')
from oracle import oracle as O  # noqa: E402


def main(out):
    out = pathlib.Path(out)
    out.mkdir(parents=True, exist_ok=True)
    floor, cells = pkg.shared_map_arrays()
    floor.tofile(out / 'floor.bin')
    cells.tofile(out / 'cells.bin')
    r = pkg.data.rays()
    np.ascontiguousarray(r['ends'], np.int8).tofile(out / 'ray_ends.bin')
    np.ascontiguousarray(r['masks'], np.uint64).tofile(out / 'ray_masks.bin')
    cfgs = [pkg.baseline_config(8), pkg.config.stress_config(), pkg.config.reference_config(24),
            pkg.config.v1_config(8), pkg.config.reference_config(8)]
    (out / 'configs.bin').write_bytes(b''.join(bytes(c) for c in cfgs))
    maps = O.LearnTablesHost([floor, O.level(3, 1), O.level(3, 2)])
    for name in ('floor', 'cells', 'index', 'distance', 'ncells', 'offsets', 'los'):
        np.ascontiguousarray(getattr(maps, name)).tofile(out / f'learn_{name}.bin')
    (out / 'learn_config.bin').write_bytes(bytes(pkg.config.learn_config()))
    print(f'asan inputs in {out}: {len(cfgs)} env configs, {maps.n_maps} learning maps, '
          f'{C.sizeof(pkg.config.D1Config)} B per config')


if __name__ == '__main__':
    main(sys.argv[1])
