"""Loads libd1hip.so (built in-tree by build.py) and declares its C ABI (include/d1hip.h).

There is no fallback: without the built library every entry point raises."""
import ctypes as C
import pathlib

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / 'libd1hip.so'
_LIB = None

SYMBOLS = ('d1_state_bytes', 'd1_obs_bytes', 'd1_action_size', 'd1_out_size', 'd1_config_bytes',
           'd1_init', 'd1_step', 'd1_heuristic', 'd1_sample', 'd1_sample_dev', 'd1_gae', 'd1_obs_to_bf16', 'd1_obs_d4',
           'd1_ppo_work_bytes', 'd1_ppo_prepare', 'd1_ppo_step', 'd1_ppo_step_static', 'd1_wait_bytes', 'd1_wait_init', 'd1_wait_run',
           'd1_sample_ar', 'd1_los_table', 'd1_distance_rows', 'd1_policy_packed_elems', 'd1_policy_pack',
           'd1_policy_fwd', 'd1_policy_fwd_sample', 'd1_policy_ar_packed_elems', 'd1_policy_ar_pack',
           'd1_policy_fwd_sample_ar')
LEARN_SYMBOLS = ('learn_turn_cost', 'learn_return_gamma', 'learn_state_bytes', 'learn_obs_size',
                 'learn_action_size', 'learn_out_size', 'learn_config_bytes', 'learn_init', 'learn_step',
                 'learn_step_active', 'learn_heuristic')
_LEARN = {}


class D1PPOStep(C.Structure):
    """The D1PPOStep struct of include/d1hip.h (one PPO minibatch update)."""
    _fields_ = [('obs', C.c_void_p), ('perm', C.c_void_p), ('cursor', C.c_void_p), ('actions', C.c_void_p),
                ('logp_old', C.c_void_p), ('adv', C.c_void_p), ('ret', C.c_void_p), ('n', C.c_int64),
                ('mb', C.c_int32), ('pad0', C.c_int32), ('p', C.c_void_p), ('pb', C.c_void_p),
                ('g', C.c_void_p), ('m', C.c_void_p), ('v', C.c_void_p), ('nparams', C.c_int64),
                ('off_w1', C.c_int64), ('off_b1', C.c_int64), ('off_w2', C.c_int64), ('off_b2', C.c_int64),
                ('off_w3', C.c_int64), ('off_b3', C.c_int64), ('step', C.c_void_p), ('loss_parts', C.c_void_p), ('work', C.c_void_p),
                ('work_bytes', C.c_int64), ('clip', C.c_float), ('vcoef', C.c_float), ('ecoef', C.c_float),
                ('max_grad_norm', C.c_float), ('lr', C.c_float), ('beta1', C.c_float), ('beta2', C.c_float),
                ('eps', C.c_float), ('z_out', C.c_void_p)]


def load():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f'{LIB_PATH} is missing: build it with __graft_entry__.build() '
                               '(the D:1 environment has no CPU fallback)')
        L = C.CDLL(str(LIB_PATH))
        p, i = C.c_void_p, C.c_int
        L.d1_state_bytes.argtypes = [i]
        for name in ('d1_obs_bytes', 'd1_action_size', 'd1_out_size', 'd1_config_bytes'):
            getattr(L, name).argtypes = []
        L.d1_init.argtypes = [p, i, i, p, p, C.c_uint64, p, p, p]
        L.d1_step.argtypes = [p, i, i, p, p, p, p, p, p, p, p]
        L.d1_heuristic.argtypes = [p, i, i, p, i, p, p]
        L.d1_sample.argtypes = [p, i, i, i, C.c_uint64, C.c_uint32, p, p, p]
        L.d1_sample_dev.argtypes = [p, i, i, i, C.c_uint64, p, C.c_uint32, p, p, p]
        L.d1_obs_to_bf16.argtypes = [p, p, C.c_int64, p]
        L.d1_obs_d4.argtypes = [p, p, i, p, p]
        L.d1_ppo_work_bytes.argtypes = [i]
        L.d1_ppo_work_bytes.restype = C.c_int64
        L.d1_ppo_step.argtypes = [C.POINTER(D1PPOStep), p]
        L.d1_ppo_prepare.argtypes = [C.POINTER(D1PPOStep), p]
        L.d1_ppo_step_static.argtypes = [C.POINTER(D1PPOStep), p]
        L.d1_sample_ar.argtypes = [p, i, i, p, i, i, i, C.c_uint64, C.c_uint32, p, p, p, p, p]
        L.d1_wait_bytes.argtypes = []
        L.d1_wait_init.argtypes = [p, i, i, p, p, C.c_uint64, i, p]
        L.d1_wait_run.argtypes = [p, i, i, p, p, i, p, p]
        L.d1_gae.argtypes = [p, p, p, p, i, i, C.c_float, C.c_float, p, p, p]
        L.d1_los_table.argtypes = [p, i, p, p, p]
        L.d1_distance_rows.argtypes = [p, p, i, p, p]
        L.d1_policy_packed_elems.argtypes = []
        L.d1_policy_packed_elems.restype = C.c_int64
        L.d1_policy_pack.argtypes = [p, p, p, p, p]
        L.d1_policy_fwd.argtypes = [p, i, p, p, p, p, p, p, p]
        L.d1_policy_fwd_sample.argtypes = [p, i, p, p, p, p, C.c_uint64, p, C.c_uint32, p, p, p, p, p]
        L.d1_policy_ar_packed_elems.argtypes = []
        L.d1_policy_ar_packed_elems.restype = C.c_int64
        L.d1_policy_ar_pack.argtypes = [p, p, p, p, p, p, p, p]
        L.d1_policy_fwd_sample_ar.argtypes = [p, i, p, p, p, p, p, C.c_uint64, p, C.c_uint32, p, p, p, p, p, p, p, p]
        _LIB = L
    return _LIB


def load_learn(clump=0):
    """libd1learn_clump{0,1}.so: the learning task's learn_* ABI (include/d1learn.h)."""
    if clump not in (0, 1):
        raise ValueError('clump mode is 0 or 1')
    if clump not in _LEARN:
        path = HERE / f'libd1learn_clump{clump}.so'
        if not path.exists():
            raise RuntimeError(f'{path} is missing: build it with __graft_entry__.build() '
                               '(the learning task has no CPU fallback)')
        L = C.CDLL(str(path))
        p, i = C.c_void_p, C.c_int
        for name in ('learn_turn_cost', 'learn_return_gamma'):
            getattr(L, name).restype = C.c_float
            getattr(L, name).argtypes = []
        for name in ('learn_state_bytes', 'learn_obs_size', 'learn_action_size', 'learn_out_size',
                     'learn_config_bytes'):
            getattr(L, name).argtypes = []
        L.learn_init.argtypes = [p, i, p, p, C.c_uint64, p, p, p, i]
        L.learn_step.argtypes = [p, i, p, p, p, i, p, p, p, p, i]
        L.learn_step_active.argtypes = [p, i, p, p, p, i, p, p, p, p, p, i]
        L.learn_heuristic.argtypes = [p, i, p, p, p, p, i]
        _LEARN[clump] = L
    return _LEARN[clump]


def check(code, what):
    if code:
        raise RuntimeError(f'{what} failed with code {code}')
