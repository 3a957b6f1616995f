"""ctypes binding of librocketnpu (MI355X) — the C-ABI exactly as include/*.h declares it.

Every function keeps its C name, argument order and integer return codes, so Python
callers (the tests, bench.py) read like the reference's C tests. Array arguments accept
numpy arrays (host memory, staged by the library), torch tensors (device memory, used in
place) or raw integer addresses.

The library must already be built (``make -C rocket-userspace_amd``); loading fails loudly
otherwise — there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "librocketnpu.so")
INCLUDE = os.path.join(REPO, "include")

ROCKET_HIP_ASYNC, ROCKET_HIP_DEVICE_OPERANDS = 1, 2
ROCKET_OK, ROCKET_E_SHAPE, ROCKET_E_TILING, ROCKET_E_NOMEM, ROCKET_E_DEVICE, ROCKET_E_UNSUPPORTED = 0, -1, -2, -3, -4, -5

i32, i64, u32, u64, sz, vp, fl = C.c_int, C.c_int64, C.c_uint32, C.c_uint64, C.c_size_t, C.c_void_p, C.c_float
ip = C.POINTER(C.c_int)
pp = C.POINTER(C.c_void_p)   # arrays of operand pointers


class RocketBO(C.Structure):
    _fields_ = [("handle", C.c_uint32), ("dma_address", C.c_uint64), ("mmap_offset", C.c_uint64),
                ("size", C.c_size_t), ("ptr", C.c_void_p)]


class RocketBORange(C.Structure):
    _fields_ = [("offset", C.c_uint64), ("size", C.c_uint64)]


class WeightsInfo(C.Structure):
    _fields_ = [("kind", u32), ("flags", u32), ("N", u32), ("K", u32), ("group", u32), ("M", u32),
                ("code_bytes", u64), ("scale_bytes", u64)]


class HwProfile(C.Structure):
    _fields_ = [("name", C.c_char_p), ("cbuf_banks", C.c_int), ("cbuf_bank_size", C.c_int),
                ("max_tile", C.c_int), ("kgroup_2b", C.c_int), ("kgroup_4b", C.c_int),
                ("ngroup", C.c_int), ("dtype_supported", C.c_uint32), ("select_warning", C.c_char_p),
                ("default_workers", C.c_int)]


class I32Stats(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("submits", "tasks", "redo_empty", "redo_zeroed", "atoms_empty",
                                         "atoms_zeroed", "accepted_zero", "refused")]


LOG_CB = C.CFUNCTYPE(None, C.c_int, C.c_char_p, C.c_void_p)
P4 = [ip, ip, ip]   # Mt, Kt, Nt out-params of the planners

# name: (restype, argtypes)
PROTOS = {
    # rocket_npu.h
    "rocket_open": (i32, []), "rocket_close": (None, [i32]),
    "rocket_affinity_set_base": (None, [i32]), "rocket_affinity_get_base": (i32, []),
    "rocket_pin_worker": (None, [i32]), "rocket_num_big_cores": (i32, []),
    "rocket_bo_alloc": (i32, [i32, sz, C.POINTER(RocketBO)]),
    "rocket_bo_free": (None, [i32, C.POINTER(RocketBO)]),
    "rocket_bo_prep": (i32, [i32, C.POINTER(RocketBO), i32, u64]),
    "rocket_bo_fini": (i32, [i32, C.POINTER(RocketBO)]),
    "rocket_bo_prep_ranges": (i32, [i32, C.POINTER(RocketBO), C.POINTER(RocketBORange), C.c_uint, u64]),
    "rocket_bo_fini_ranges": (i32, [i32, C.POINTER(RocketBO), C.POINTER(RocketBORange), C.c_uint]),
    "rocket_bo_ranges_supported": (i32, []), "rocket_batched_submit_supported": (i32, []),
    "rocket_ppu_done_supported": (i32, []), "rocket_batch_completion_tracked": (i32, []),
    "rocket_busy_poll_set_us": (None, [C.c_long]),
    "rocket_submit_matmul": (i32, [i32, C.POINTER(RocketBO), u32, vp, u32, vp, u32, u32]),
    "rocket_submit_matmul_flags": (i32, [i32, C.POINTER(RocketBO), u32, vp, u32, vp, u32, u32]),
    "rocket_submit_tasks": (i32, [i32, vp, u32, vp, u32, vp, u32]),
    "rocket_submit_tasks_flags": (i32, [i32, vp, u32, vp, u32, vp, u32, u32]),
    "rocket_submit_scratch_size": (sz, [u32]),
    "rocket_submit_tasks_pre": (i32, [i32, vp, vp, u32, vp, u32, vp, u32, u32]),
    "rocket_submit_jobs": (i32, [i32, vp, u32]),
    "rocket_submit_ioctl_count": (u64, []), "rocket_submit_task_count": (u64, []),
    "rocket_submit_counters_reset": (None, []),
    # rocket_log.h
    "rocket_log_set_callback": (None, [LOG_CB, vp]), "rocket_log_set_level": (None, [i32]),
    "rocket_log_get_level": (i32, []), "rocket_log": (None, [i32, C.c_char_p]),
    # rocket_hw_profile.h
    "rocket_hw_current": (C.POINTER(HwProfile), []), "rocket_hw_by_name": (C.POINTER(HwProfile), [C.c_char_p]),
    # rocket_matmul.h — planners
    "rocket_matmul_plan": (i32, [i32, i32, i32] + P4), "rocket_matmul_plan_int8": (i32, [i32, i32, i32] + P4),
    "rocket_matmul_plan_int8_gw": (i32, [i32, i32, i32, i32] + P4), "rocket_matmul_plan_int4": (i32, [i32, i32, i32] + P4),
    "rocket_matmul_plan_int16": (i32, [i32, i32, i32] + P4), "rocket_matmul_plan_bf16": (i32, [i32, i32, i32] + P4),
    "rocket_matmul_plan_tf32": (i32, [i32, i32, i32] + P4), "rocket_matmul_plan_int8_rk3576": (i32, [i32, i32, i32] + P4),
    # one-shot entries
    "rocket_matmul_fp16": (i32, [i32, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_fp16_f32out": (i32, [i32, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_fp16_batch": (i32, [i32, i32, i32, i32, i32, pp, pp, pp]),
    "rocket_mm_batch_create": (vp, [i32]), "rocket_mm_batch_free": (None, [vp]),
    "rocket_mm_batch_run": (i32, [vp, i32, i32, i32, i32, pp, pp, pp]),
    "rocket_matmul_int8": (i32, [i32, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_int8_groupwise": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, i32]),
    "rocket_matmul_int4": (i32, [i32, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_int4_ex": (i32, [i32, i32, i32, i32, vp, vp, vp, i32]),
    "rocket_matmul_int4_groupwise": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, i32]),
    "rocket_matmul_int16_exact": (i32, [i32, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_bf16": (i32, [i32, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_bf16_mt": (i32, [i32, i32, i32, vp, vp, vp, i32]),
    "rocket_bf16_stream_create": (vp, [i32]), "rocket_bf16_stream_free": (None, [vp]),
    "rocket_matmul_bf16_stream": (i32, [vp, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_tf32": (i32, [i32, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_fp16_mt": (i32, [i32, i32, i32, vp, vp, vp, i32]),
    # RK3576 stubs
    "rocket_matmul_int8_rk3576": (i32, [i32, i32, i32, i32, vp, vp, vp, fl, vp]),
    "rocket_matmul_int8_rk3576_perc": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, vp]),
    "rocket_matmul_int8_rk3576_perc_sa": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp]),
    "rocket_rk3576_wbo_create": (i32, [i32, i32, i32, vp, C.POINTER(C.c_void_p)]),
    "rocket_rk3576_wbo_free": (None, [i32, vp]),
    "rocket_matmul_int8_rk3576_perc_wbo": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp]),
    "rocket_rk3576_bo_pool_drain": (None, [i32]),
    "rocket_matmul_int8_rk3576_i32": (i32, [i32, i32, i32, i32, vp, vp, vp, vp]),
    "rocket_rk3576_i32_last_stats": (None, [C.POINTER(I32Stats)]),
    # resident fp16 / streams
    "rocket_ctx_create": (vp, [i32]), "rocket_ctx_free": (None, [vp]),
    "rocket_weights_pack": (vp, [vp, i32, i32, i32, vp]), "rocket_weights_free": (None, [vp, vp]),
    "rocket_matmul_fp16_prepacked": (i32, [vp, i32, i32, i32, vp, vp, vp]),
    "rocket_stream_create": (vp, [i32]), "rocket_stream_free": (None, [vp]),
    "rocket_matmul_fp16_stream": (i32, [vp, i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_fp16_stream_fused": (i32, [vp, i32, i32, pp, ip, i32, vp, vp]),
    # resident int8 / int4
    "rocket_i8_ctx_create": (vp, [i32]), "rocket_i8_ctx_free": (None, [vp]),
    "rocket_i8_weights_pack": (vp, [vp, i32, i32, i32, vp]), "rocket_i8_weights_free": (None, [vp, vp]),
    "rocket_i8_weights_bytes": (sz, [vp]),
    "rocket_matmul_int8_prepacked": (i32, [vp, i32, i32, i32, vp, vp, vp]),
    "rocket_i8_weights_pack_gw": (vp, [vp, i32, i32, i32, vp, i32]),
    "rocket_matmul_int8_prepacked_gw": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp]),
    "rocket_i4_ctx_create": (vp, [i32]), "rocket_i4_ctx_free": (None, [vp]),
    "rocket_i4_weights_pack": (vp, [vp, i32, i32, i32, vp]), "rocket_i4_weights_free": (None, [vp, vp]),
    "rocket_matmul_int4_prepacked": (i32, [vp, i32, i32, i32, vp, vp, vp]),
    "rocket_i4_weights_pack_gw": (vp, [vp, i32, i32, i32, vp, i32]),
    "rocket_matmul_int4_prepacked_gw": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp]),
    "rocket_i4_weights_bytes": (sz, [vp]),
    # rocket_hip.h (MI355X additions)
    "rocket_hip_stream": (vp, [i32]), "rocket_hip_set_stream": (i32, [i32, vp]),
    "rocket_hip_set_mode": (i32, [i32, C.c_uint]), "rocket_hip_sync": (i32, [i32]),
    "rocket_ctx_fd": (i32, [vp]), "rocket_i8_ctx_fd": (i32, [vp]), "rocket_i4_ctx_fd": (i32, [vp]),
    "rocket_stream_fd": (i32, [vp]), "rocket_bf16_stream_fd": (i32, [vp]),
    "rocket_matmul_int8_groupwise_dump": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, i32, i32, i32, vp]),
    "rocket_matmul_int4_groupwise_dump": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, i32, i32, i32, vp]),
    "rocket_matmul_int8_prepacked_gw_dump": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp, i32, i32, vp]),
    "rocket_matmul_int4_prepacked_gw_dump": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp, i32, i32, vp]),
    "rocket_matmul_int8_prepacked_gw_grouped": (i32, [vp, i32, ip, i32, i32, pp, pp, pp, pp, pp]),
    "rocket_matmul_int8_prepacked_gw_rowscale_dump": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp, i32, i32, vp]),
    "rocket_matmul_int4_prepacked_gw_rowscale_dump": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp, i32, i32, vp]),
    "rocket_matmul_int8_prepacked_gw_grouped_dump": (i32, [vp, i32, ip, i32, i32, pp, pp, pp, pp, pp, ip, ip, pp]),
    "rocket_matmul_int8_prepacked_gw_grouped_rowscale_dump": (i32, [vp, i32, ip, i32, i32, pp, pp, pp, pp, pp, ip, ip,
                                                                    pp]),
    "rocket_matmul_int8_groupwise_rowscale": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, i32]),
    "rocket_matmul_int4_groupwise_rowscale": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, vp, i32]),
    "rocket_matmul_int8_prepacked_gw_rowscale": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp]),
    "rocket_matmul_int4_prepacked_gw_rowscale": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp]),
    "rocket_matmul_int8_prepacked_gw_grouped_rowscale": (i32, [vp, i32, ip, i32, i32, pp, pp, pp, pp, pp]),
    "rocket_i8_weights_device": (vp, [vp]), "rocket_i4_weights_device": (vp, [vp]),
    # rocket_ffn.h
    "rocket_geglu_fp16": (i32, [i32, vp, vp, i32, vp, i32]),
    "rocket_geglu_ref_fp16": (None, [vp, vp, i32, vp, i32]),
    "rocket_ffn_fp16": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    "rocket_ffn_ref_fp16": (None, [i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    "rocket_ffn_fp16_fused": (i32, [i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    "rocket_mlp_fp16_fused": (i32, [i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    # rocket_attn.h
    "rocket_mha_self_fp16": (i32, [i32, i32, i32, i32] + [vp] * 10),
    "rocket_mha_self_ref_fp16": (None, [i32, i32, i32] + [vp] * 10),
    "rocket_fa_ctx_create": (vp, [i32]),
    "rocket_fa_ctx_free": (None, [vp]),
    "rocket_flash_attn_fp16": (i32, [i32] + [i32] * 6 + [fl, fl] + [vp] * 5),
    "rocket_flash_attn_fp16_mt": (i32, [i32] + [i32] * 6 + [fl, fl] + [vp] * 5 + [i32]),
    "rocket_flash_attn_fp16_ctx": (i32, [vp] + [i32] * 6 + [fl, fl] + [vp] * 5),
    "rocket_flash_attn_ref_fp16": (None, [i32] * 6 + [fl, fl] + [vp] * 5),
    # rocket_weights_io.h
    "rocket_weights_info_read": (i32, [vp, sz, vp]),
    "rocket_weights_xxh64": (u64, [vp, sz]),
    "rocket_i8_weights_serialized_bytes": (sz, [vp, i32]),
    "rocket_i4_weights_serialized_bytes": (sz, [vp, i32]),
    "rocket_i8_weights_serialize": (C.c_long, [vp, vp, vp, vp, sz]),
    "rocket_i4_weights_serialize": (C.c_long, [vp, vp, vp, vp, sz]),
    "rocket_i8_weights_deserialize": (vp, [vp, vp, sz, vp]),
    "rocket_i4_weights_deserialize": (vp, [vp, vp, sz, vp]),
    "rocket_i8_weights_save": (i32, [vp, vp, vp, C.c_char_p]),
    "rocket_i4_weights_save": (i32, [vp, vp, vp, C.c_char_p]),
    "rocket_i8_weights_load": (vp, [vp, C.c_char_p, vp]),
    "rocket_i4_weights_load": (vp, [vp, C.c_char_p, vp]),
    # rocket_quant.h
    "rocket_quantize_rows_int8": (i32, [i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_int4_prepacked_gw_f32in_noalloc": (i32, [vp, i32, i32, i32, vp, vp, vp, vp]),
    "rocket_quantize_rows_int8_fp16": (i32, [i32, i32, i32, vp, vp, vp]),
    "rocket_matmul_int8_prepacked_gw_f32in": (i32, [vp, i32, i32, i32, vp, vp, vp, vp]),
    "rocket_matmul_int4_prepacked_gw_f32in": (i32, [vp, i32, i32, i32, vp, vp, vp, vp]),
    "rocket_matmul_int8_prepacked_gw_grouped_f32in": (i32, [vp, i32, ip, i32, i32, pp, pp, pp, pp]),
    "rocket_matmul_int8_prepacked_gw_grouped_glu_f32in": (i32, [vp, i32, ip, i32, i32, pp, pp, i32, pp, pp, pp]),
    "rocket_matmul_int8_prepacked_gw_grouped_glu_f16in": (i32, [vp, i32, ip, i32, i32, pp, pp, i32, pp, pp, pp]),
    "rocket_matmul_int8_prepacked_gw_grouped_rowscale_f16out": (i32, [vp, i32, ip, i32, i32, pp, pp, pp, pp, pp]),
}

# rocket_activation.h
ROCKET_ACTIVATION_SILU, ROCKET_ACTIVATION_TANH, ROCKET_ACTIVATION_GELU = 3, 4, 5

# data objects exported by the headers (not functions)
DATA_SYMBOLS = ("rocket_hw_mi355x", "rocket_hw_rk3588", "rocket_hw_rk3576")

_lib = None


def _share_torch_runtime():
    """PyTorch-ROCm bundles its own HIP runtime, which its libraries NEED by the unversioned
    name libamdhip64.so. If librocketnpu (NEEDED libamdhip64.so.7) is loaded first, torch
    later maps a second HIP runtime into the process and finds no GPU. Importing torch
    first makes the loader satisfy librocketnpu's libamdhip64.so.7 with torch's copy (same
    SONAME), so the process keeps one runtime. ROCKETNPU_NO_TORCH=1 skips this."""
    if os.environ.get("ROCKETNPU_NO_TORCH") == "1":
        return
    try:
        import torch  # noqa: F401
    except Exception:
        pass


def load(path: str | None = None) -> C.CDLL:
    """Load librocketnpu.so and declare every prototype. Raises when it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(f"librocketnpu.so is not built ({p}); run `make -C {HERE}`")
    _share_torch_runtime()
    lib = C.CDLL(p)
    for name, (res, args) in PROTOS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    if path is None:
        _lib = lib
    return lib


def header_functions() -> list[str]:
    """Every function name declared in include/*.h (parsed from the headers)."""
    names = set()
    pat = re.compile(r"^[A-Za-z_][\w\s\*]*?\b(rocket_\w+)\s*\(", re.M)
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for line in text.splitlines():
            line = line.strip()
            if line.startswith(("#", "typedef", "return", "//")) or "static inline" in line:
                continue
            m = pat.match(line)
            if m:
                names.add(m.group(1))
    return sorted(names)


# ---- argument helpers ---------------------------------------------------------------

def ptr(x):
    """Address of a numpy array / torch tensor / int (None -> NULL)."""
    if x is None:
        return None
    if isinstance(x, int):
        return C.c_void_p(x)
    if hasattr(x, "data_ptr"):        # torch.Tensor
        return C.c_void_p(x.data_ptr())
    if hasattr(x, "ctypes"):          # numpy.ndarray
        if not x.flags["C_CONTIGUOUS"]:
            raise ValueError("operand must be C-contiguous")
        return C.c_void_p(x.ctypes.data)
    raise TypeError(f"cannot take the address of {type(x)}")


def ptr_array(xs):
    arr = (C.c_void_p * len(xs))()
    for i, x in enumerate(xs):
        p = ptr(x)
        arr[i] = p.value if p is not None else None
    return C.cast(arr, pp), arr   # keep `arr` alive while the call runs


def int_array(xs):
    arr = (C.c_int * len(xs))(*xs)
    return C.cast(arr, ip), arr


def plan(fn: str, *dims):
    """Call a planner; returns (count, Mt, Kt, Nt)."""
    lib = load()
    mt, kt, nt = C.c_int(0), C.c_int(0), C.c_int(0)
    r = getattr(lib, fn)(*dims, C.byref(mt), C.byref(kt), C.byref(nt))
    return r, mt.value, kt.value, nt.value
