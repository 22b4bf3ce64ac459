"""ctypes binding of libhipenvs.so and the tensor checks shared by every module.

The library is the product: every env step and rollout runs in it. Nothing here
computes a result on the host; when the library is missing or no GPU is
visible, the call raises instead of falling back to anything else.

torch is imported before the library is opened so that the process holds one
HIP runtime: libhipenvs.so's ``libamdhip64.so.7`` dependency binds to the
runtime torch already loaded, and torch's stream handles are valid for it.
"""

import contextlib
import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).with_name("libhipenvs.so")

OK, E_ARG, E_UNSUPPORTED, E_HIP, E_SCRATCH = 0, -1, -2, -3, -4

# bytes of the static device array behind hipenvs_es_update_static (HIPENVS_ES_UPDATE_STATIC_BYTES)
ES_UPDATE_STATIC_BYTES = 2 * 1024 * 1024

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_F32 = ctypes.c_float

# name -> argtypes, every entry point of include/hipenvs.h that returns a status int
SIGNATURES = {
    "hipenvs_cartpole_reset": [_P, _I64, _U32, _P],
    "hipenvs_cartpole_step": [_P, _P, _U32, _P, _P, _P, _I64, _P],
    "hipenvs_cartpole_step_k": [_P, _P, _U32, _I32, _P, _P, _P, _I64, _P],
    "hipenvs_sample_actions": [_P, _I64, _I32, _U32, _P],
    "hipenvs_detmath": [_P, _P, _P, _P, _I64, _P],
    "hipenvs_div_recip": [_P, _P, _P, _P, _I64, _P],
    "hipenvs_sqrt_recip_check": [_U64, _U64, _P, _P],
    "hipenvs_cartpole_es_rollout": [_P, _P, _I64, _I32, _I32, _P, _P],
    "hipenvs_acrobot_reset": [_P, _I64, _U32, _P],
    "hipenvs_acrobot_step": [_P, _P, _U32, _P, _P, _P, _I64, _P],
    "hipenvs_acrobot_es_rollout": [_P, _P, _I64, _I32, _I32, _P, _P],
    "hipenvs_pendulum_aba_reset": [_I32, _I32, _P, _I64, _U32, _P],
    "hipenvs_pendulum_aba_step": [_I32, _P, _P, _U32, _P, _P, _P, _I64, _P],
    "hipenvs_pendulum_aba_step_euler": [_I32, _P, _P, _U32, _P, _P, _P, _I64, _P],
    "hipenvs_pendulum_aba_accelerations": [_I32, _P, _P, _P, _I64, _P],
    "hipenvs_legged_reset": [_I32, _P, _P, _I64, _U32, _P],
    "hipenvs_legged_step": [_I32, _I32, ctypes.c_double, _P, _P, _U32, _P, _P, _P, _P, _I64, _P],
    "hipenvs_legged_step_reference": [_I32, _I32, ctypes.c_double, _P, _I32, _P, _U32, _P, _P, _P, _P, _I64, _P],
    "hipenvs_legged_es_rollout": [_I32, _I32, _I32, _I32, _P, _P, _I64, _I32, _F32, _F32, _F32, ctypes.c_double,
                                  _P, _P, _P],
    "hipenvs_legged_es_rollout_chunked": [_I32, _I32, _I32, _I32, _P, _P, _I64, _I32, _F32, _F32, _F32,
                                          ctypes.c_double, _P, _P, _P, _I64, _P],
    "hipenvs_legged_es_rollout_chunked_rows": [_I32, _I32, _I32, _I32, _P, _P, _I64, _I32, _F32, _F32, _F32,
                                               ctypes.c_double, _P, _P, _P, _I64, _P],
    "hipenvs_pendulum_step": [_I32, _P, _P, _U32, _P, _P, _P, _I64, _P],
    "hipenvs_pendulum_accelerations": [_I32, _P, _P, _P, _I64, _P],
    "hipenvs_hopper_reset": [_P, _I64, _U32, _P],
    "hipenvs_hopper_step": [_P, _P, _U32, _P, _P, _P, _I64, _P],
    "hipenvs_cartpole_evaluate": [_P, _P, _I64, _I32, _I32, _P, _P],
    "hipenvs_acrobot_evaluate": [_P, _P, _I64, _I32, _I32, _P, _P],
    "hipenvs_legged_evaluate": [_I32, _I32, _I32, _P, _P, _I64, _I32, _F32, _P, _P],
    "hipenvs_es_perturb": [_P, _I64, _I64, _U32, ctypes.c_double, _I32, _P, _P],
    "hipenvs_es_update": [_P, _P, _I64, _I64, _U32, ctypes.c_double, ctypes.c_double, _P, _P, _I64, _P],
    "hipenvs_es_update_static": [_P, _P, _I64, _I64, _U32, ctypes.c_double, ctypes.c_double, _P, _P],
    "hipenvs_cartpole_es_rollout_seeded": [_P, _P, _I64, _U32, ctypes.c_double, _I32, _I32, _P, _P, _I64, _P],
    "hipenvs_acrobot_es_rollout_seeded": [_P, _P, _I64, _U32, ctypes.c_double, _I32, _I32, _P, _P, _I64, _P],
    "hipenvs_legged_es_rollout_seeded": [_I32, _I32, _I32, _I32, _P, _P, _I64, _U32, ctypes.c_double, _I32, _F32,
                                         _F32, _F32, ctypes.c_double, _P, _P, _P, _I64, _P],
}

# entry points that return a value rather than a status
VALUE_SIGNATURES = {
    "hipenvs_legged_es_rollout_workspace_bytes": (ctypes.c_int64, [_I32, _I32, _I64]),
    "hipenvs_es_update_workspace_bytes": (ctypes.c_int64, [_I64, _I64]),
}


class HipEnvsError(RuntimeError):
    """A failed hipenvs call: bad argument, unsupported shape, or a HIP launch error."""


_lib = None


def lib():
    """The loaded library; raises HipEnvsError when it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HipEnvsError(f"{LIB_PATH} is missing; build it with `python metal-rl-envs_amd/build.py`")
        handle = ctypes.CDLL(str(LIB_PATH))
        handle.hipenvs_version.restype = ctypes.c_char_p
        handle.hipenvs_version.argtypes = []
        handle.hipenvs_last_hip_error.restype = ctypes.c_int
        handle.hipenvs_last_hip_error.argtypes = []
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        for name, (restype, argtypes) in VALUE_SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def call(name, *args):
    """Call entry point `name` and raise HipEnvsError on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != OK:
        if rc == E_HIP:
            raise HipEnvsError(f"{name}: HIP launch failed (hipError_t {lib().hipenvs_last_hip_error()})")
        if rc == E_UNSUPPORTED:
            raise HipEnvsError(f"{name}: no kernel instantiated for these compile-time parameters")
        if rc == E_SCRATCH:
            raise HipEnvsError(f"{name}: the shape needs more than the library's static scratch holds")
        raise HipEnvsError(f"{name}: invalid argument (status {rc})")


def version():
    return lib().hipenvs_version().decode()


# ---- tensor plumbing --------------------------------------------------------

def default_device():
    if not torch.cuda.is_available():
        raise HipEnvsError("hipenvs needs a ROCm GPU: torch.cuda.is_available() is False")
    return torch.device("cuda", torch.cuda.current_device())


# torch's own accessors of the current raw stream and device, which skip building a Stream
# object (about 1.5 us a call) and the device context's exchange (about 1 us); the public
# forms stand in where an older torch lacks them
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)
_NO_SWITCH = contextlib.nullcontext()


def stream_of(device):
    """hipStream_t handle (an int, which ctypes passes as a pointer) of torch's current
    stream on `device`."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def on(device):
    """A context in which `device` is the current device; nothing to switch when it already is."""
    if _get_device is not None and device.index is not None and _get_device() == device.index:
        return _NO_SWITCH
    return torch.cuda.device(device)


def ptr(t):
    """Device address of tensor `t` as an int (None, passed as NULL, for no tensor)."""
    return t.data_ptr() if t is not None else None


def check_state(state, rows, name="state", dtypes=(torch.float32,)):
    """A (rows, n) contiguous tensor on a GPU of one of `dtypes` (float32 by default); returns n."""
    if not isinstance(state, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(state).__name__}")
    if state.dtype not in dtypes:
        names = " or ".join(str(d).replace("torch.", "") for d in dtypes)
        raise TypeError(f"{name} must be {names}, got {state.dtype}")
    if state.dim() != 2 or state.shape[0] != rows:
        raise ValueError(f"{name} must have shape ({rows}, n), got {tuple(state.shape)}")
    if state.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm GPU, got device {state.device}")
    if not state.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return state.shape[1]


def as_actions(action, n, device, name="action"):
    """An (n,) int32 contiguous device tensor; other integer dtypes are converted (one copy)."""
    if not isinstance(action, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(action).__name__}")
    if action.dtype.is_floating_point or action.dtype == torch.bool or action.dtype.is_complex:
        raise TypeError(f"{name} must be an integer tensor, got {action.dtype}")
    if action.shape != (n,):
        raise ValueError(f"{name} must have shape ({n},), got {tuple(action.shape)}")
    if action.device != device:
        raise ValueError(f"{name} is on {action.device}, state is on {device}")
    if action.dtype != torch.int32:
        action = action.to(torch.int32)
    return action.contiguous()


def as_f32_vector(x, n, device, name):
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(x).__name__}")
    if x.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {x.dtype}")
    if x.shape != (n,):
        raise ValueError(f"{name} must have shape ({n},), got {tuple(x.shape)}")
    if x.device != device:
        raise ValueError(f"{name} is on {x.device}, state is on {device}")
    return x.contiguous()


def u32(seed):
    return ctypes.c_uint32(int(seed) & 0xFFFFFFFF)


# ---- shared launch helpers of the step and rollout modules -------------------

def launch_reset(entry, rows, n, seed, device):
    """A fresh (rows, n) state from reset entry point `entry` at counter `seed`."""
    state = torch.empty((rows, n), dtype=torch.float32, device=device)
    with on(device):
        call(entry, ptr(state), n, u32(seed), stream_of(device))
    return state


def launch_step(entry, rows, state, action, seed, *extra):
    """(next_state, reward, done) of step entry point `entry`; `extra` C arguments go
    between the seed and the output pointers."""
    n = check_state(state, rows)
    device = state.device
    action = as_actions(action, n, device)
    next_state = torch.empty_like(state)
    reward = torch.empty(n, dtype=torch.float32, device=device)
    done = torch.empty(n, dtype=torch.bool, device=device)
    with on(device):
        call(entry, ptr(state), ptr(action), u32(seed), *extra, ptr(next_state), ptr(reward), ptr(done), n,
             stream_of(device))
    return next_state, reward, done


def check_theta(theta_pop, p, d, device, name="theta_pop"):
    """A (p, d) float32 contiguous device tensor (es.unflatten's row layout)."""
    if not isinstance(theta_pop, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(theta_pop).__name__}")
    if theta_pop.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {theta_pop.dtype}")
    if theta_pop.shape != (p, d):
        raise ValueError(f"{name} must have shape ({p}, {d}), got {tuple(theta_pop.shape)}")
    if theta_pop.device != device:
        raise ValueError(f"{name} is on {theta_pop.device}, state is on {device}")
    return theta_pop.contiguous()


HIDDEN_SIZES = (4, 8, 16, 32, 64)


def check_hidden(hidden):
    if int(hidden) not in HIDDEN_SIZES:
        raise ValueError(f"hidden must be one of {HIDDEN_SIZES}, got {hidden}")
    return int(hidden)


def check_horizon(horizon):
    if int(horizon) < 0:
        raise ValueError("horizon must be >= 0")
    return int(horizon)


def check_population(p):
    """An even population of at least 2 (antithetic pairs)."""
    p = int(p)
    if p < 2 or p % 2:
        raise ValueError(f"the population must be even and at least 2 (antithetic pairs), got {p}")
    return p


def check_theta_vector(theta, d, device, name="theta"):
    """The (d,) float32 contiguous device tensor of the unperturbed parameters."""
    if not isinstance(theta, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(theta).__name__}")
    if theta.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {theta.dtype}")
    if theta.shape != (d,):
        raise ValueError(f"{name} must have shape ({d},), got {tuple(theta.shape)}")
    if theta.device != device:
        raise ValueError(f"{name} is on {theta.device}, state is on {device}")
    return theta.contiguous()
