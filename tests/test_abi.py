"""The C-ABI library loads and exports every symbol include/d1hip.h declares (no GPU needed)."""
import ctypes as C
import re

import pytest

from conftest import ROOT


def declared_symbols():
    text = (ROOT / 'include' / 'd1hip.h').read_text()
    return sorted(set(re.findall(r'^\w[\w\s\*]*?\b(d1_\w+)\s*\(', text, re.M)))


def test_header_declares_the_abi():
    assert declared_symbols() == sorted(['d1_state_bytes', 'd1_obs_bytes', 'd1_action_size', 'd1_out_size',
                                         'd1_config_bytes', 'd1_init', 'd1_step', 'd1_sample', 'd1_gae',
                                         'd1_obs_to_bf16', 'd1_ppo_gather', 'd1_ppo_loss', 'd1_relu_bwd',
                                         'd1_adam_clip', 'd1_relu_bwd_bias', 'd1_colsum',
                                         'd1_sum_partials', 'd1_wait_bytes', 'd1_wait_init', 'd1_wait_run',
                                         'd1_sample_ar'])


def test_library_exports_declared_symbols(pkg):
    lib = pytest.importorskip('importlib').import_module('dcss-auto_amd._lib').load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.d1_obs_bytes() == 1800 and lib.d1_action_size() == 19 and lib.d1_out_size() == 8
    assert lib.d1_config_bytes() == C.sizeof(pkg.D1Config)
    assert lib.d1_state_bytes(8) == 2688 and lib.d1_state_bytes(40) == 2944
    assert lib.d1_state_bytes(0) < 0 and lib.d1_state_bytes(65) < 0


def test_argument_validation_without_gpu(pkg):
    """Rejected configs return negative codes before any launch."""
    L = pytest.importorskip('importlib').import_module('dcss-auto_amd._lib').load()
    cfg = pkg.baseline_config()
    tab = pkg.D1Tables(None, None, None, 11)
    assert L.d1_init(None, 4, 8, C.byref(cfg), C.byref(tab), 0, None, None, None) == -1   # no ray table
    tab = pkg.D1Tables(None, None, 1, 11)
    bad = pkg.baseline_config(9)
    assert L.d1_init(1, 4, 8, C.byref(bad), C.byref(tab), 0, None, None, None) == -2     # count > capacity
    shared = pkg.reference_config()
    assert L.d1_init(1, 4, 40, C.byref(shared), C.byref(tab), 0, None, None, None) == -1  # shared map missing
    assert L.d1_step(1, 0, 8, C.byref(cfg), C.byref(tab), 1, None, None, None, None, None) == 0  # empty batch
