"""The C-ABI libraries load and export every symbol include/d1hip.h and include/d1learn.h
declare (no GPU needed)."""
import ctypes as C
import re

import pytest

from conftest import ROOT


def declared_symbols(header='d1hip.h', prefix='d1_'):
    text = (ROOT / 'include' / header).read_text()
    return sorted(set(re.findall(r'^\w[\w\s\*]*?\b(' + prefix + r'\w+)\s*\(', text, re.M)))


def test_header_declares_the_abi():
    assert declared_symbols() == sorted(['d1_state_bytes', 'd1_obs_bytes', 'd1_action_size', 'd1_out_size',
                                         'd1_config_bytes', 'd1_init', 'd1_step', 'd1_heuristic', 'd1_sample', 'd1_sample_dev', 'd1_gae',
                                         'd1_obs_to_bf16', 'd1_obs_d4', 'd1_ppo_work_bytes', 'd1_ppo_prepare', 'd1_ppo_step',
                                         'd1_ppo_step_static',
                                         'd1_wait_bytes', 'd1_wait_init', 'd1_wait_run',
                                         'd1_sample_ar', 'd1_los_table', 'd1_distance_rows', 'd1_policy_packed_elems',
                                         'd1_policy_pack', 'd1_policy_fwd', 'd1_policy_fwd_sample',
                                         'd1_policy_ar_packed_elems', 'd1_policy_ar_pack', 'd1_policy_fwd_sample_ar'])
    # the reference's learn_* exports (gpu-d1/branches/d1-stairs-v2/src/learn.cu:913-946)
    assert declared_symbols('d1learn.h', 'learn_') == sorted(
        ['learn_turn_cost', 'learn_return_gamma', 'learn_state_bytes', 'learn_obs_size', 'learn_action_size',
         'learn_out_size', 'learn_config_bytes', 'learn_init', 'learn_step', 'learn_step_active',
         'learn_heuristic'])


@pytest.mark.parametrize('clump', [0, 1])
def test_learn_library_exports(pkg, clump):
    import importlib
    _lib = importlib.import_module('dcss-auto_amd._lib')
    lib = _lib.load_learn(clump)
    for name in declared_symbols('d1learn.h', 'learn_'):
        assert hasattr(lib, name), name
    assert sorted(_lib.LEARN_SYMBOLS) == declared_symbols('d1learn.h', 'learn_')
    assert (lib.learn_obs_size(), lib.learn_action_size(), lib.learn_out_size()) == (1015, 19, 45)
    assert lib.learn_config_bytes() == C.sizeof(pkg.config.D1LConfig) == 140
    assert lib.learn_state_bytes() == 13184
    assert lib.learn_turn_cost() == pytest.approx(1e-5) and lib.learn_return_gamma() == 1.0
    cfg = pkg.config.learn_config()
    tab = pkg.config.D1LTables(1, 1, None, None, 836, 1, None, 1, -1, 1)
    assert lib.learn_init(1, 4, C.byref(cfg), C.byref(tab), 0, None, None, None, 0) == -3   # no host path
    assert lib.learn_init(1, 4, C.byref(pkg.config.learn_config(23)), C.byref(tab), 0, None, None, None, 1) == -2
    nolos = pkg.config.D1LTables(1, 1, None, None, 836, 1, None, 1, -1, None)
    assert lib.learn_step(1, 4, C.byref(cfg), C.byref(nolos), 1, 2048, None, None, None, None, 1) == -1
    assert lib.learn_step(1, 0, C.byref(cfg), C.byref(tab), 1, 2048, None, None, None, None, 1) == 0


def test_learn_config_packing(pkg):
    """The reference wrapper's int array (learn_env_ring_multi.py:93-97) and the struct agree."""
    cfg = pkg.config.learn_config()
    words = list((C.c_int32 * 35).from_buffer_copy(bytes(cfg)))
    assert words[:11] == [24, 3631, 18, 681, 794, 906, 2, 23, 1, 25, 26]   # gdr: 393216^(1/4), 458752^(1/4)
    assert words[11:15] == [10, 3, 19, 15]


def test_library_exports_declared_symbols(pkg):
    lib = pytest.importorskip('importlib').import_module('dcss-auto_amd._lib').load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.d1_obs_bytes() == 1800 and lib.d1_action_size() == 19 and lib.d1_out_size() == 8
    assert lib.d1_config_bytes() == C.sizeof(pkg.D1Config)
    assert lib.d1_state_bytes(8) == 2688 and lib.d1_state_bytes(40) == 5696   # 40: + the distance-field memo
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
    assert L.d1_heuristic(1, 4, 8, C.byref(bad), 1, 1, None) == -1                  # count > capacity
    assert L.d1_heuristic(1, 4, 8, C.byref(cfg), 2, 1, None) == -1                  # joint is 0 or 1
    assert L.d1_heuristic(None, 4, 8, C.byref(cfg), 1, 1, None) == -1               # no state
    assert L.d1_heuristic(1, 0, 8, C.byref(cfg), 1, 1, None) == 0                   # empty batch


def test_ppo_step_struct_layout(tmp_path):
    """The ctypes D1PPOStep and the C struct agree field by field (gcc on the header)."""
    import importlib
    import subprocess
    _lib = importlib.import_module('dcss-auto_amd._lib')
    names = [f for f, _ in _lib.D1PPOStep._fields_]
    src = tmp_path / 'layout.c'
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "d1hip.h"\nint main(void) {\n'
                   '  printf("%zu\\n", sizeof(D1PPOStep));\n' +
                   ''.join(f'  printf("%zu\\n", offsetof(D1PPOStep, {f}));\n' for f in names) + '  return 0;\n}\n')
    exe = tmp_path / 'layout'
    subprocess.run(['gcc', '-I', str(ROOT / 'include'), '-o', str(exe), str(src)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert got[0] == C.sizeof(_lib.D1PPOStep)
    assert got[1:] == [getattr(_lib.D1PPOStep, f).offset for f in names]


def test_ppo_step_validation_without_gpu(pkg):
    """Workspace sizing and rejected PPO arguments need no GPU."""
    import importlib
    _lib = importlib.import_module('dcss-auto_amd._lib')
    L = _lib.load()
    assert L.d1_ppo_work_bytes(1000) == -1 and L.d1_ppo_work_bytes(0) == -1
    w8k = L.d1_ppo_work_bytes(8192)
    # 4 activation/gradient arrays [256][mb] + dz [17][mb] (bf16), bias partials, split-K partials
    assert w8k >= 4 * 256 * 8192 * 2 + 8 * 256 * 1800 * 4
    assert L.d1_ppo_work_bytes(4096) < w8k
    assert L.d1_ppo_step(None, None) == -1 and L.d1_ppo_prepare(None, None) == -1
    s = _lib.D1PPOStep(mb=1000, n=4096)
    assert L.d1_ppo_step(C.byref(s), None) == -1                  # minibatch not a multiple of 1024
    s = _lib.D1PPOStep(mb=1024, n=512)
    assert L.d1_ppo_step(C.byref(s), None) == -1                  # fewer samples than one minibatch
    s = _lib.D1PPOStep(mb=1024, n=4096)
    assert L.d1_ppo_step(C.byref(s), None) == -1                  # null buffers


def test_policy_fwd_validation_without_gpu(pkg):
    """Packed-weight sizing and rejected forward arguments need no GPU."""
    import importlib
    _lib = importlib.import_module('dcss-auto_amd._lib')
    L = _lib.load()
    # W1 [8][29 chunks][4][64][8] + W2 [8][16][64][8] + head [16][64][8]
    assert L.d1_policy_packed_elems() == 8 * 29 * 4 * 512 + 8 * 16 * 512 + 16 * 512
    assert L.d1_policy_pack(None, None, None, None, None) == -1
    assert L.d1_policy_fwd(None, 0, None, None, None, None, None, None, None) == 0      # empty batch
    assert L.d1_policy_fwd(None, -1, None, None, None, None, None, None, None) == -1
    assert L.d1_policy_fwd(None, 4, None, None, None, None, None, None, None) == -1     # null buffers
    fake = 1 << 20
    assert L.d1_policy_fwd(fake + 4, 4, fake, fake, fake, fake, fake, fake, None) == -1   # obs not 8-byte aligned
    assert L.d1_policy_fwd(fake, 4, fake + 8, fake, fake, fake, fake, fake, None) == -1   # packed weights not 16-byte aligned
    assert L.d1_policy_fwd(fake, 4, fake, fake, fake, fake, fake + 4, fake, None) == -1   # logits not 16-byte aligned
    # the autoregressive head's region after it: two t1 tiles [2][16][64][8], t2 [4][64][8], ev [8][64]
    assert L.d1_policy_ar_packed_elems() == L.d1_policy_packed_elems() + 2 * 16 * 512 + 4 * 512 + 8 * 64
    assert L.d1_policy_ar_pack(None, None, None, None, None, None, None, None) == -1
    args = [fake, 4, fake, fake, fake, fake, fake, 0, None, 0, fake, fake, fake, None, None, None, None, None]
    assert L.d1_policy_fwd_sample_ar(*args[:1], 0, *args[2:]) == 0                       # empty batch
    for k, bad in ((0, fake + 4), (2, fake + 8), (6, fake + 2), (15, fake + 4), (10, None), (11, None)):
        a = list(args)
        a[k] = bad                                                                     # misaligned or missing
        assert L.d1_policy_fwd_sample_ar(*a) == -1, k


def test_missing_library_raises(monkeypatch, tmp_path):
    """No CPU fallback: with the HIP library absent, loading it (what every entry point does
    first) raises and names the build step."""
    import importlib
    L = importlib.import_module('dcss-auto_amd._lib')
    monkeypatch.setattr(L, '_LIB', None)
    monkeypatch.setattr(L, 'LIB_PATH', tmp_path / 'libd1hip.so')
    with pytest.raises(RuntimeError, match='no CPU fallback'):
        L.load()
    monkeypatch.setattr(L, '_LEARN', {})
    monkeypatch.setattr(L, 'HERE', tmp_path)
    with pytest.raises(RuntimeError, match='no CPU fallback'):
        L.load_learn(1)
