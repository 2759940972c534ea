"""ctypes binding of libacfun_amd.so (the C ABI declared in include/acfun/acfun.h).

The same signature table binds any library exporting the reference's acfun_*
API, which is what lets tests drive this library and the reference through
identical calls.  Loading fails loudly when the built library is missing:
there is no CPU fallback behind these entry points.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libacfun_amd.so")

_i, _f, _sz, _p = C.c_int, C.c_float, C.c_size_t, C.c_void_p
_s = C.c_char_p

# name -> (restype, argtypes); pointer arguments are void* so numpy arrays
# (arr.ctypes.data) and device addresses (int) both pass.
SIGNATURES = {
    # reference public API (acfun.h:15-148 of the reference)
    "acfun_set_threads": (None, [_i]),
    "acfun_backend": (_i, []),
    "acfun_backend_name": (_s, []),
    "acfun_autotune": (None, []),
    "acfun_tune_status": (_s, []),
    "acfun_gemm": (None, [_i, _i, _i, _p, _p, _p]),
    "acfun_gemm_epi": (None, [_i, _i, _i, _p, _p, _p, _p, _i]),
    "acfun_gemm_bf16": (None, [_i, _i, _i, _p, _p, _p]),
    "acfun_conv2d": (None, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _i, _i, _i, _p]),
    "acfun_conv2d_relu": (None, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _i, _i, _i, _p]),
    "acfun_conv2d_dw": (None, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _i, _i, _p, _i]),
    "acfun_conv2d_g": (None, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p, _i]),
    "acfun_fc": (None, [_p, _i, _i, _p, _p, _i, _p]),
    "acfun_fc_relu": (None, [_p, _i, _i, _p, _p, _i, _p]),
    "acfun_relu": (None, [_p, _sz]),
    "acfun_relu6": (None, [_p, _sz]),
    "acfun_maxpool": (None, [_p, _i, _i, _i, _i, _i, _i, _i, _p]),
    "acfun_maxpool_relu": (None, [_p, _i, _i, _i, _i, _i, _i, _i, _p]),
    "acfun_softmax": (None, [_p, _i, _i, _p]),
    "acfun_batchnorm": (None, [_p, _i, _i, _p, _p, _p, _p, _f]),
    "acfun_quantize_weights": (None, [_p, _i, _i, _p, _p]),
    "acfun_conv2d_int8": (None, [_p, _i, _i, _i, _i, _p, _p, _p, _i, _i, _i, _i, _i, _f, _p, _i]),
    "acfun_model_load": (_p, [_s]),
    "acfun_model_destroy": (None, [_p]),
    "acfun_model_infer": (_i, [_p, _p, _p]),
    "acfun_model_output_size": (_i, [_p]),
    "acfun_model_input_dims": (None, [_p, _p, _p, _p]),
    # reference internal entry points its tests bind (src/internal.h)
    "acfun_gemm_int8": (None, [_i, _i, _i, _p, _p, _p]),
    "acfun_gemm_int8_epi": (None, [_i, _i, _i, _p, _p, _p, _p, _p, _i]),
    "acfun_quantize_u8": (None, [_p, _p, _sz, _f, _i]),
    "acfun_conv2d_int8_direct": (None, [_p, _i, _i, _i, _i, _p, _p, _p, _i, _i, _i, _i, _i,
                                        _i, _i, _p, _i]),
    "acfun_conv1x1_int8": (None, [_p, _i, _i, _i, _p, _p, _p, _p, _i]),
    "acfun_winograd_conv3x3_int8": (None, [_p, _i, _i, _i, _i, _p, _p, _p, _i, _f, _f, _p, _i]),
    "acfun_winograd_conv3x3": (None, [_p, _i, _i, _i, _i, _p, _p, _i, _p, _i]),
    "acfun_winograd43_conv3x3": (None, [_p, _i, _i, _i, _i, _p, _p, _i, _p, _i]),
    "acfun_conv2d_grouped": (None, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p, _i]),
    "acfun_set_num_threads_runtime": (None, [_i]),
    "acfun_get_num_threads_runtime": (_i, []),
    "acfun_effective_cores": (_i, []),
    # new in this library
    "acfun_last_error": (_s, []),
    "acfun_sync": (_i, []),
    "acfun_dev_gemm_epi": (_i, [_i, _i, _i, _p, _p, _p, _p, _i, _p]),
    "acfun_dev_gemm_bf16": (_i, [_i, _i, _i, _p, _p, _p, _p]),
    "acfun_dev_conv2d": (_i, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p, _i, _p]),
    "acfun_dev_conv2d_int8": (_i, [_p, _i, _i, _i, _i, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i,
                                   _p]),
    "acfun_dev_conv2d_int8_q": (_i, [_p, _p, _i, _i, _i, _i, _p, _p, _p, _i, _i, _i, _i, _i,
                                     _p, _p, _i, _i, _p]),
    "acfun_dev_conv2d_int8_noalloc": (_i, [_p, _i, _i, _i, _i, _p, _p, _p, _i, _i, _i, _i, _i,
                                           _p, _i, _p]),
    "acfun_dev_conv2d_dw_maxpool": (_i, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _i, _i, _i, _i, _i,
                                         _i, _p, _i, _p]),
    "acfun_dev_conv2d_g_maxpool": (_i, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _i, _i, _i, _i, _i,
                                        _i, _i, _i, _p, _i, _p]),
    "acfun_dev_maxpool": (_i, [_p, _i, _i, _i, _i, _i, _i, _i, _p, _i, _p]),
    "acfun_dev_fc": (_i, [_p, _i, _i, _p, _p, _i, _p, _i, _p]),
    "acfun_dev_softmax": (_i, [_p, _i, _i, _p, _p]),
    "acfun_model_load_ex": (_p, [_s, _i]),
    "acfun_model_infer_batch": (_i, [_p, _i, _p, _p]),
    "acfun_dev_model_infer_batch": (_i, [_p, _i, _p, _p, _p]),
    "acfun_prof_enable": (None, [_i]),
    "acfun_prof_kernel_ms": (C.c_double, [_s, C.POINTER(_i)]),
    "acfun_prof_report": (_i, [C.c_char_p, _i]),
}


def bind(cdll, required=None):
    """Sets restype/argtypes on every table entry the library exports.

    `required` (an iterable of names) raises AttributeError when one is absent.
    """
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(cdll, name, None)
        if fn is None:
            if required is not None and name in required:
                raise AttributeError(f"{name} missing from {cdll._name}")
            continue
        fn.restype = res
        fn.argtypes = args
    return cdll


_lib = None


def lib():
    """The product library (raises when it has not been built).

    torch is imported first when it is installed: it bundles its own HIP
    runtime under the same soname (libamdhip64.so.7) as the ROCm one this
    library links, and the first one loaded serves the whole process.  Loading
    torch's first keeps one runtime in the process, so torch tensors and this
    library share devices, streams and allocations.
    """
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              "`python -c 'import __graft_entry__ as g; g.build()'`")
        _lib = bind(C.CDLL(LIB_PATH), required=SIGNATURES.keys())
    return _lib


def prof_report():
    """acfun_prof_report as (kernels, layers): kernels maps (tag, name) to
    (launches, total ms); layers is a list of per-layer dicts."""
    L = lib()
    n = L.acfun_prof_report(None, 0)
    if n < 0:
        raise RuntimeError(last_error())
    buf = C.create_string_buffer(n)
    if L.acfun_prof_report(buf, n) < 0:
        raise RuntimeError(last_error())
    kernels, layers = {}, []
    keys = ("i", "type", "N", "H", "W", "C", "OH", "OW", "OC", "KH", "KW", "stride", "pad",
            "groups", "int8", "fused_into", "act", "residual")
    for ln in buf.value.decode().splitlines():
        f = ln.split("\t")
        if f[0] == "K":
            kernels[(int(f[1]), f[2])] = (int(f[3]), float(f[4]))
        elif f[0] == "L":
            layers.append(dict(zip(keys, map(int, f[1:]))))
    return kernels, layers


def last_error():
    e = lib().acfun_last_error()
    return e.decode() if e else ""
