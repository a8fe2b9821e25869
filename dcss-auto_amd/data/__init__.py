"""Static data: the LOS ray table and map 1057, derived by make_data.py."""
import functools
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent


@functools.lru_cache(None)
def rays():
    with np.load(HERE / 'los_rays.npz') as f:
        return {k: f[k] for k in f.files}


@functools.lru_cache(None)
def map1057():
    with np.load(HERE / 'map1057.npz') as f:
        return {k: f[k] for k in f.files}
