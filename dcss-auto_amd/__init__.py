"""d1hip: MI355X-native batched DCSS D:1 environment, policy sampling, GAE and PPO.

The package directory name contains a hyphen, so import it with
``importlib.import_module('dcss-auto_amd')``.
"""
from . import data  # noqa: F401
from .config import (D1Config, D1Tables, baseline_config, make_config, reference_config,  # noqa: F401
                     shared_map_arrays, stress_config, v1_config)
from .env import Env  # noqa: F401,E402
