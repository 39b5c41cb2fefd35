"""ctypes binding of libtcacomp.so (include/tca_rt.h + include/tca_cg.h).

The library is built in-tree by ``tcacomp_amd.build.build_library()``.
Loading fails loudly when it is missing: there is no Python fallback for
any part of the compile or launch path.
"""
import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# TCA_LIB names another build of the same library (the sanitizer gate loads
# tcacomp_amd/_asan/libtcacomp.so, built with AddressSanitizer and UBSan).
LIB_PATH = os.environ.get("TCA_LIB") or os.path.join(PKG_DIR, "libtcacomp.so")

TCA_MAX_RANK = 8

# Status codes (tca_rt.h).
TCA_OK = 0
TCA_ERR_INVALID = 1
TCA_ERR_SHAPE = 2
TCA_ERR_LAUNCH = 3
TCA_ERR_HIP = 4
TCA_ERR_NOT_FOUND = 5
TCA_ERR_UNSUPPORTED = 6
TCA_ERR_BUILD = 7


class tca_tensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("rank", ctypes.c_uint32),
        ("dims", ctypes.c_uint32 * TCA_MAX_RANK),
        ("dtype", ctypes.c_int32),
    ]


class tca_operand(ctypes.Structure):
    _fields_ = [
        ("tensor", ctypes.c_int32),
        ("rank", ctypes.c_uint32),
        ("axes", ctypes.c_int32 * TCA_MAX_RANK),
    ]


class tca_device_info(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("compute_units", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("max_threads_per_block", ctypes.c_int32),
        ("max_lds_per_block", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("total_global_mem", ctypes.c_uint64),
    ]


# (name, restype, argtypes) for every exported entry point.
_c = ctypes
_P = _c.c_void_p
_I32 = _c.c_int32
_U32 = _c.c_uint32
_STR = _c.c_char_p
SIGNATURES = [
    # runtime (tca_rt.h)
    ("tca_rt_last_error", _STR, []),
    ("tca_rt_init", _c.c_int, [_c.c_int]),
    ("tca_rt_device_info", _c.c_int, [_c.c_int, _c.POINTER(tca_device_info)]),
    ("tca_rt_device_sync", _c.c_int, []),
    ("tca_rt_malloc", _c.c_int, [_c.POINTER(_P), _c.c_size_t]),
    ("tca_rt_free", _c.c_int, [_P]),
    ("tca_rt_memcpy_h2d", _c.c_int, [_P, _P, _c.c_size_t]),
    ("tca_rt_memcpy_d2h", _c.c_int, [_P, _P, _c.c_size_t]),
    ("tca_rt_memset", _c.c_int, [_P, _c.c_int, _c.c_size_t]),
    ("tca_rt_stream_create", _c.c_int, [_c.POINTER(_P)]),
    ("tca_rt_stream_destroy", _c.c_int, [_P]),
    ("tca_rt_stream_sync", _c.c_int, [_P]),
    ("tca_rt_event_create", _c.c_int, [_c.POINTER(_P)]),
    ("tca_rt_event_destroy", _c.c_int, [_P]),
    ("tca_rt_event_record", _c.c_int, [_P, _P]),
    ("tca_rt_event_elapsed_ms", _c.c_int, [_P, _P, _c.POINTER(_c.c_float)]),
    ("tca_rt_module_load", _c.c_int, [_STR, _c.POINTER(_P)]),
    ("tca_rt_module_unload", _c.c_int, [_P]),
    ("tca_rt_validate_launch", _c.c_int, [_U32, _U32, _U32]),
    ("tca_rt_launch", _c.c_int, [_P, _STR, _U32, _U32, _U32, _P, _c.c_size_t, _P]),
    ("tca_program_load", _c.c_int, [_STR, _STR, _c.POINTER(_P)]),
    ("tca_program_unload", _c.c_int, [_P]),
    ("tca_program_parse", _c.c_int, [_STR, _c.POINTER(_P)]),
    ("tca_program_signature", _c.c_int,
     [_P, _c.POINTER(_U32), _c.POINTER(_U32), _c.POINTER(_U32), _c.POINTER(_U32)]),
    ("tca_program_check", _c.c_int,
     [_P, _c.POINTER(tca_tensor), _U32, _c.POINTER(_U32), _U32]),
    ("tca_program_selected", _c.c_int,
     [_P, _c.POINTER(tca_tensor), _U32, _c.POINTER(_U32), _U32, _c.POINTER(_c.c_uint8),
      _c.POINTER(_c.c_uint64), _c.POINTER(_U32), _U32]),
    ("tca_program_launch", _c.c_int,
     [_P, _c.POINTER(tca_tensor), _U32, _c.POINTER(_U32), _U32, _c.POINTER(_c.c_double), _U32, _P]),
    ("tca_program_launch_noalloc", _c.c_int,
     [_P, _c.POINTER(tca_tensor), _U32, _c.POINTER(_U32), _U32, _c.POINTER(_c.c_double), _U32, _P]),
    ("tca_program_kernel_name", _STR, [_P, _U32]),
    ("tca_program_plan_text", _STR, [_P]),
    ("tca_program_kernel_args", _I32, [_P, _P, _U32, _P, _U32, _P, _U32, _U32, _P, _c.c_size_t, _P]),
    # builder + emitter (tca_cg.h)
    ("tca_builder_new", _P, [_STR]),
    ("tca_builder_free", None, [_P]),
    ("tca_builder_error", _STR, [_P]),
    ("tca_builder_dim", _I32, [_P, _STR, _c.c_int64]),
    ("tca_builder_tensor", _I32, [_P, _STR, _I32, _U32, _c.POINTER(_I32)]),
    ("tca_builder_local", _I32, [_P, _STR, _I32, _U32, _c.POINTER(_I32)]),
    ("tca_builder_scalar", _I32, [_P, _STR, _I32]),
    ("tca_expr_const", _I32, [_P, _I32, _c.c_double]),
    ("tca_expr_binop", _I32, [_P, _I32, _I32, _I32]),
    ("tca_expr_unop", _I32, [_P, _I32, _I32]),
    ("tca_expr_select", _I32, [_P, _I32, _I32, _I32]),
    ("tca_expr_cast", _I32, [_P, _I32, _I32]),
    ("tca_expr_call", _I32, [_P, _STR, _U32, _c.POINTER(_I32)]),
    ("tca_expr_error", _STR, [_P, _I32]),
    ("tca_expr_dtype", _I32, [_P, _I32]),
    ("tca_stmt", _I32, [_P]),
    ("tca_chain_iter", _c.c_int, [_P, _I32, _U32, _c.POINTER(_I32)]),
    ("tca_chain_map_begin", _c.c_int,
     [_P, _I32, _U32, _c.POINTER(tca_operand), _c.POINTER(_I32), _c.POINTER(_U32)]),
    ("tca_chain_map_end", _c.c_int, [_P, _I32, _I32]),
    ("tca_chain_as", _c.c_int, [_P, _I32, _U32, _c.POINTER(_I32)]),
    ("tca_chain_reduce_begin", _c.c_int, [_P, _I32, _I32, _c.POINTER(_I32), _c.POINTER(_I32)]),
    ("tca_chain_reduce_end", _c.c_int, [_P, _I32, _I32]),
    ("tca_chain_store", _c.c_int, [_P, _I32, _I32, _U32, _c.POINTER(_I32)]),
    ("tca_builder_build", _c.c_int, [_P]),
    ("tca_builder_ir", _STR, [_P]),
    ("tca_builder_ir_full", _STR, [_P]),
    ("tca_emit", _c.c_int, [_P, _STR, _STR, _I32, _c.POINTER(_P)]),
    ("tca_emit_source", _STR, [_P]),
    ("tca_emit_plan", _STR, [_P]),
    ("tca_emit_report", _STR, [_P]),
    ("tca_emit_hipcc_argc", _U32, [_P]),
    ("tca_emit_hipcc_arg", _STR, [_P, _U32]),
    ("tca_emit_free", None, [_P]),
    # .tca frontend (tca_syntax.h)
    ("tca_syntax_parse_module", _c.c_int, [_STR, _c.POINTER(_P)]),
    ("tca_syntax_parse_source", _c.c_int, [_STR, _STR, _I32, _c.POINTER(_P)]),
    ("tca_syntax_last_error", _STR, []),
    ("tca_syntax_module_diagnostics", _STR, [_P]),
    ("tca_syntax_module_kernel_count", _U32, [_P]),
    ("tca_syntax_module_kernel_name", _STR, [_P, _U32]),
    ("tca_syntax_module_kernel_cxx_name", _STR, [_P, _U32]),
    ("tca_syntax_module_runtime_path", _STR, [_P]),
    ("tca_syntax_module_dump", _STR, [_P]),
    ("tca_syntax_module_build_kernel", _c.c_int, [_P, _U32, _c.POINTER(_P)]),
    ("tca_syntax_module_free", None, [_P]),
]

_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                "libtcacomp.so is not built (%s); run tcacomp_amd.build.build_library() "
                "or __graft_entry__.build()" % LIB_PATH)
        l = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def last_error():
    msg = lib().tca_rt_last_error()
    return msg.decode() if msg else ""


class TcaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("tca error %d: %s" % (code, msg))
        self.code = code


def check(rc):
    if rc != TCA_OK:
        raise TcaError(rc, last_error())
