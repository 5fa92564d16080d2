"""The C ABI of include/noise_amd.h as ctypes declarations: entry-point signatures, result types, structs and
flag values. Free of torch, so that tools which only call the library's host layer (argument checks,
error messages) can load it on its own."""
import ctypes

_p, _i64, _u64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, ctypes.c_float

# name -> argtypes (every entry point returns int status unless listed in _RESTYPES)
SIGNATURES = {
    'noise_abi_version': [],
    'noise_last_error': [],
    'noise_draw_layout': [_i32, _i64, _p, _p],
    'noise_normal_fill': [_p, _i64, _i64, _u64, _u64, _i64, _f32, _f32, _p],
    'noise_randint': [_p, _i64, _u64, _u64, _i64, _u64, _i64, _p],
    'noise_gather_slices': [_p, _i64, _i64, _p, _p, _i64, _u64, _u64, _i64, _p],
    'noise_gather_slice_groups': [_p, _i64, _i64, _p, _p, _i64, _u64, _u64, _i64, _p],
    'noise_orthogonal_draws': [_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _p],
    'noise_attention_fwd': [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i64, _i64, _i64, _i32, _i64, _i64, _i64, _i64, _f32, _p, _i64, _i64, _p, _p],
    'noise_v_transpose': [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p],
    'noise_pop_embed': [_p, _i32, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p],
    'noise_member_dots': [_p, 'View', _i64, _p, _i64, _p, _p],
    'noise_pop_qkv': [_p, 'View', _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _p, _p, _p],
    'noise_pop_gate': [_p, 'View', _p, _p, _p, _p],
    'noise_pop_qkv_shared': [_p, _p, _p, _p, _p, _p, _p, _p],
    'noise_pop_residual': [_p, 'View', _p, _i64, _p, _p, _i64, _i64, 'View', _p, _i32, _p, _p, _p, _p,
                           _i64, 'View', _p, _i32, _p, _i64, _p, _p],
    'noise_pop_fc': [_p, 'View', _p, _p, _p, _p, _p, _p, _p],
    'noise_pop_mlp': [_p, 'View', _p, _p, _p, _p, _p, 'View', _p, _i32, _p, _p, _p, _p, _i64, 'View', _p, _i32, _p,
                      _i64, _p, _p],
    'noise_pop_attn_mlp': [_p, 'View', _p, _p, _p, _i64, 'View', _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _i64,
                           'View', _p, _i32, _p, _i64, _p, _p],
    'noise_pop_block': [_p, 'View', _p, _p, _p, _i64, 'View', _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _i64,
                        'View', _p, _i32, _p, _i64, _p, _p],
    'noise_pop_block_qkv': [_p, 'View', _p, _p, _p, _i64, 'View', _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _i64,
                            'View', _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _p, _p, _p, _p],
    'noise_block_weight_layout': [_p, _p, _i64, _i64, _p],
    'noise_mlp_proj_layout': [_p, _p, _i64, _p],
    'noise_pop_linear': [_p, 'View', _p, _i64, _i64, _p, _p, _p, _i32, _i64, _i64, _p],
    'noise_pop_head_ce': [_p, 'View', _p, _i64, _i64, _p, _p, _p, _i64, _p, _p],
    'noise_member_mean': [_p, _i64, _i64, _p, _p],
    'noise_split3': [_p, _i64, _i64, _i32, _i32, _p, _p],
    'noise_lowrank_embed': [_p, _p, _i64, _i64, _p, _p, _p, _p],
    'noise_rank1_expand': [_p, _p, _i64, _p, _i64, _p, _p, _i32, _p],
    'noise_lowrank_rows': [_p, 'View', _i64, _p, _i64, _p, _p, _p],
    'noise_coordinate_differences': [_p, _i32, _i64, _i64, _i64, _p, _f32, _p, _i64, _i64, _p],
    'noise_draw_errors': [_p, _p, _i64, _i64, _i64, _f32, _p, _p],
    'noise_rerun_rows': [_p, _i64, _p, _p, _i64, _p, _p, _i64, _p, _p],
    'noise_rerun_mix_norm': [_p, _i64, _p, _i64, _p, _p, _i64, _p, _p, _p],
    'noise_block_entry': [_p, _i64, _p, _i64, _p, _p, _p],
    'noise_add_bf16': [_p, _p, _i64, _p],
    'noise_mask_scale': [_p, _p, _i64, _i64, _f32, _p, _p],
    'noise_pop_block_jit': [_p, 'View', _p, 'View', _p, _p, _i32, _p, _p, 'View', _p, _i32, _p, _p],
    'noise_pop_block_qkv_jit': [_p, 'View', _p, 'View', _p, _p, _p, _p, _p, 'View', _p, _p, _p, _p, _i64, _p, _i64, _p,
                                _p, _p, _p],
    'noise_dust_block_workspace_bytes': [_i64, _i64, _i32],
    'noise_dust_block': [_p, _p, _i64, _i64, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _i64, _p],
    'noise_dust_block_static_max_bytes': [],
    'noise_dust_block_static': [_p, _p, _i64, _i64, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p],
    'noise_update_weights': [_p, _i64, _i64, _p, _p],
    'noise_update_workspace_bytes': [_p, _i32, _i64, _i64],
    'noise_update_gradients': [_p, _i32, _i64, _p, _f32, _i64, _i64, _u64, _u64, _i64, _p, _p, _i64, _p],
}
_RESTYPES = {'noise_last_error': ctypes.c_char_p, 'noise_update_workspace_bytes': ctypes.c_int64,
             'noise_dust_block_workspace_bytes': ctypes.c_int64, 'noise_dust_block_static_max_bytes': ctypes.c_int64}

# y_fp32 of noise_pop_linear / noise_rank1_expand: fp32 output in autocast's form (bf16 product and dot)
LINEAR_AUTOCAST = 2

# noise_population_t.rounding (include/noise_amd.h)
ROUNDING_FUSED = 0
ROUNDING_EAGER = 1

# noise_attention_fwd flags (include/noise_amd.h)
ATTN_V_TRANSPOSED = 1
ATTN_QK_NORMED = 2


class View(ctypes.Structure):
    """noise_view_t: element (m, t, j) at ptr + m*sm + t*st + j."""
    _fields_ = [('ptr', ctypes.c_void_p), ('sm', ctypes.c_int64), ('st', ctypes.c_int64)]


class Rank1(ctypes.Structure):
    """noise_rank1_t: per-direction a [dirs, out], b [dirs, in] rows (NULL a: unperturbed)."""
    _fields_ = [('a', ctypes.c_void_p), ('b', ctypes.c_void_p), ('a_stride', ctypes.c_int64),
                ('b_stride', ctypes.c_int64)]


class Population(ctypes.Structure):
    """noise_population_t (rounding: ROUNDING_FUSED, the default, or ROUNDING_EAGER)."""
    _fields_ = [('members', ctypes.c_int64), ('tokens', ctypes.c_int64), ('sign', ctypes.c_void_p),
                ('dir_div', ctypes.c_int64), ('rounding', ctypes.c_int64)]


SLICE_GROUPS_MAX = 64  # NOISE_SLICE_GROUPS_MAX


class SliceGroups(ctypes.Structure):
    """noise_slice_groups_t: up to 64 parameters' [pairs] offsets, widths and output columns."""
    _fields_ = [('count', ctypes.c_int32), ('offsets', ctypes.c_void_p * SLICE_GROUPS_MAX),
                ('width', ctypes.c_int64 * SLICE_GROUPS_MAX), ('col', ctypes.c_int64 * SLICE_GROUPS_MAX)]


class BlockJitter(ctypes.Structure):
    """noise_block_jitter_t: bf16 jitter rows added to mlp.c_fc's and mlp.c_proj's products (NULL: none)."""
    _fields_ = [('fc', ctypes.c_void_p), ('mlp', ctypes.c_void_p), ('zero_row', ctypes.c_void_p)]


class UpdateParam(ctypes.Structure):
    """noise_update_param_t: a parameter's [pairs] noise offsets and its fp32 gradient [rows][cols]."""
    _fields_ = [('offsets', ctypes.c_void_p), ('grad', ctypes.c_void_p), ('rows', ctypes.c_int64),
                ('cols', ctypes.c_int64)]


def bind(handle):
    """Set argtypes and restype of every entry point on a loaded libnoise_amd (ctypes.CDLL)."""
    for name, argtypes in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = [View if a == 'View' else a for a in argtypes]
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    return handle
