"""CPU oracle for the acfun convolution/GEMM path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker or the CPU baseline; the product package
(acfun_amd) never imports it.

Two libraries live here:
  * build/libacfun_oracle.so -- acfun_oracle.c, a plain-C restatement of the
    reference arithmetic (each function cites the reference file:line);
  * _ref/libacfun_ref.so     -- the reference compiled from its own sources by
    ref.mk (present wherever it was built; it is the "reference" CPU baseline).
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(_HERE, "build", "libacfun_oracle.so")
REF_SO = os.path.join(_HERE, "_ref", "libacfun_ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i, _f, _sz, _vp = C.c_int, C.c_float, C.c_size_t, C.c_void_p

_lib = None
_ref = None


def lib():
    """The C restatement (raises if it was not built: run `make -C oracle`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise FileNotFoundError(f"{ORACLE_SO} missing: run `make -C oracle`")
        L = C.CDLL(ORACLE_SO)
        sig = {
            "oracle_gemm": [_i, _i, _i, _f32p, _f32p, _f32p],
            "oracle_gemm_epi": [_i, _i, _i, _f32p, _f32p, _f32p, _vp, _i],
            "oracle_gemm_f64": [_i, _i, _i, _f32p, _f32p, _f64p],
            "oracle_bf16_round": [_f32p, _f32p, _sz],
            "oracle_conv2d_route": [_i] * 10,
            "oracle_conv2d_f64": [_f32p, _i, _i, _i, _i, _f32p, _vp, _i, _i, _i, _i, _i, _i, _f64p, _i],
            "oracle_conv2d_dw": [_f32p, _i, _i, _i, _i, _f32p, _vp, _i, _i, _i, _i, _f32p, _i],
            "oracle_conv2d_grouped": [_f32p, _i, _i, _i, _i, _f32p, _vp, _i, _i, _i, _i, _i, _i, _f32p, _i],
            "oracle_maxpool": [_f32p, _i, _i, _i, _i, _i, _i, _i, _f32p, _i],
            "oracle_relu": [_f32p, _sz],
            "oracle_relu6": [_f32p, _sz],
            "oracle_softmax": [_f32p, _i, _i, _f32p],
            "oracle_batchnorm": [_f32p, _i, _i, _f32p, _f32p, _vp, _vp, _f],
            "oracle_fold_bn": [_f32p, _f32p, _i, _i, _sz, _i, _f32p, _f32p, _f32p, _f32p],
            "oracle_quantize_weights": [_f32p, _i, _i, _f32p, _i8p],
            "oracle_absmax": [_f32p, _sz],
            "oracle_quantize_u8": [_f32p, _u8p, _sz, _f, _i, _i],
            "oracle_gemm_int8": [_i, _i, _i, _u8p, _i8p, _i32p],
            "oracle_gemm_int8_epi": [_i, _i, _i, _u8p, _i8p, _f32p, _f32p, _f32p, _i],
            "oracle_conv1x1_int8": [_u8p, _i, _i, _i, _i8p, _f32p, _f32p, _f32p, _i],
            "oracle_conv2d_int8_direct": [_u8p, _i, _i, _i, _i, _i8p, _f32p, _f32p,
                                          _i, _i, _i, _i, _i, _i, _i, _f32p, _i],
            "oracle_winograd_conv3x3_int8": [_f32p, _i, _i, _i, _i, _i8p, _f32p, _vp, _i,
                                             _f, _f, _f32p, _i],
            "oracle_conv_int8_centered_acc": [_u8p, _i, _i, _i, _i, _i8p, _i, _i, _i, _i, _i,
                                              _i, _i, _i32p],
            "oracle_conv2d_int8_route": [_i] * 8,
            "oracle_conv2d_int8": [_f32p, _i, _i, _i, _i, _i8p, _f32p, _vp, _i, _i, _i, _i, _i,
                                   _f, _f32p, _i],
            "oracle_requantize_s8": [_f32p, _sz, _i8p],
            "oracle_wino_int8_epilogue": [_i32p, _sz, _i, _f, _f32p, _vp, _f32p, _i],
            "oracle_conv2d_int8_q": [_i8p, _f, _i, _i, _i, _i, _i8p, _f32p, _vp, _i, _i, _i, _i,
                                     _i, _i8p, C.POINTER(_f), _i, _i],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        L.oracle_conv2d_route.restype = _i
        L.oracle_conv2d_int8_route.restype = _i
        L.oracle_absmax.restype = _f
        L.oracle_requantize_s8.restype = _f
        _lib = L
    return _lib


def ref():
    """The compiled reference library, or None where it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        _ref = C.CDLL(REF_SO)
    return _ref


def ptr(a):
    """ctypes void* of a numpy array, or None for None (a NULL bias)."""
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def out_hw(H, W, KH, KW, stride, pad):
    return (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1


# ---- numpy-level wrappers (shapes as the reference API takes them) ----------

def gemm(A, B):
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float32)
    lib().oracle_gemm(M, N, K, A, B, Cm)
    return Cm


def gemm_epi(A, B, bias, act):
    """acfun_gemm_ref_epi's arithmetic: i-k-j float accumulation, then +bias[j]
    and ReLU once after the full reduction."""
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float32)
    lib().oracle_gemm_epi(M, N, K, np.ascontiguousarray(A, np.float32),
                          np.ascontiguousarray(B, np.float32), Cm, ptr(bias), act)
    return Cm


def gemm_f64(A, B):
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float64)
    lib().oracle_gemm_f64(M, N, K, A, B, Cm)
    return Cm


def bf16(x):
    """x rounded to bf16 as acfun_gemm_bf16 rounds its operands, widened back to fp32."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().oracle_bf16_round(x.reshape(-1), y.reshape(-1), x.size)
    return y


def gemm_bf16_f64(A, B):
    """acfun_gemm_bf16's arithmetic in f64 (src/gemm_bf16_avx512.cpp:123-168):
    its 16 x 16 micro-tiles multiply bf16-rounded operands; rows past the last
    multiple of 16 of M and columns past the last multiple of 16 of N (its
    256 x 128 tiles are multiples of 16) take the scalar fp32 path
    (acfun_gemm_ref_ld) on the unrounded operands."""
    M, N = A.shape[0], B.shape[1]
    Cm = gemm_f64(bf16(A), bf16(B))
    M16, N16 = M // 16 * 16, N // 16 * 16
    if M16 < M:
        Cm[M16:] = gemm_f64(np.ascontiguousarray(A[M16:]), B)
    if N16 < N and M16 > 0:
        Cm[:M16, N16:] = gemm_f64(np.ascontiguousarray(A[:M16]), np.ascontiguousarray(B[:, N16:]))
    return Cm


def conv2d_f64(x, w, b, KH, KW, Cout, stride, pad, groups=1, act=0):
    N, H, W, Cin = x.shape
    OH, OW = out_hw(H, W, KH, KW, stride, pad)
    out = np.zeros((N, max(OH, 0), max(OW, 0), Cout), np.float64)
    lib().oracle_conv2d_f64(x, N, H, W, Cin, w, ptr(b), KH, KW, Cout, stride, pad, groups, out, act)
    return out


def conv2d_dw(x, w, b, KH, KW, stride, pad, act):
    N, H, W, Cc = x.shape
    OH, OW = out_hw(H, W, KH, KW, stride, pad)
    out = np.zeros((N, OH, OW, Cc), np.float32)
    lib().oracle_conv2d_dw(x, N, H, W, Cc, w, ptr(b), KH, KW, stride, pad, out, act)
    return out


def conv2d_grouped(x, w, b, KH, KW, Cout, stride, pad, groups, act):
    N, H, W, Cin = x.shape
    OH, OW = out_hw(H, W, KH, KW, stride, pad)
    out = np.zeros((N, OH, OW, Cout), np.float32)
    lib().oracle_conv2d_grouped(x, N, H, W, Cin, w, ptr(b), KH, KW, Cout, stride, pad, groups, out, act)
    return out


def maxpool(x, pool, stride, pad, post_relu=0):
    N, H, W, Cc = x.shape
    OH, OW = out_hw(H, W, pool, pool, stride, pad)
    out = np.zeros((N, OH, OW, Cc), np.float32)
    lib().oracle_maxpool(x, N, H, W, Cc, pool, stride, pad, out, post_relu)
    return out


def quantize_weights(w2d):
    K, N = w2d.shape
    s = np.empty(N, np.float32)
    q = np.empty((K, N), np.int8)
    lib().oracle_quantize_weights(np.ascontiguousarray(w2d, np.float32), K, N, s, q)
    return s, q


def quantize_u8(x, inv_s, zp=128, mode=0):
    xf = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(xf.size, np.uint8)
    lib().oracle_quantize_u8(xf, out, xf.size, inv_s, zp, mode)
    return out.reshape(np.shape(x))


def gemm_int8(A, B):
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.int32)
    lib().oracle_gemm_int8(M, N, K, A, B, Cm)
    return Cm


def gemm_int8_epi(A, B, alpha, beta, act):
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float32)
    lib().oracle_gemm_int8_epi(M, N, K, A, B, Cm, alpha, beta, act)
    return Cm


def conv2d_int8(x, wq, ws, b, KH, KW, Cout, stride, pad, act, s_in=0.0):
    N, H, W, Cin = x.shape
    OH, OW = out_hw(H, W, KH, KW, stride, pad)
    out = np.zeros((N, max(OH, 0), max(OW, 0), Cout), np.float32)
    lib().oracle_conv2d_int8(x, N, H, W, Cin, wq, ws, ptr(b), KH, KW, Cout, stride, pad,
                             s_in, out, act)
    return out


def requantize_s8(y):
    """(q, scale): the build-defined int8 output of a float tensor,
    q = clamp(RNE(y*127/max|y|), -128, 127), scale = max|y|/127 (0 for an all-zero y)."""
    yf = np.ascontiguousarray(y, np.float32).ravel()
    q = np.empty(yf.size, np.int8)
    s = lib().oracle_requantize_s8(yf, yf.size, q)
    return q.reshape(np.shape(y)), np.float32(s)


def quantize_wino_u8(x, inv_s):
    """The int8 Winograd route's input quantization: half-away-by-add on
    16-channel chunks, lroundf on the channel tail (src/winograd_int8.cpp:306-325)."""
    x = np.ascontiguousarray(x, np.float32)
    Cin = x.shape[-1]
    cvec = Cin & ~15
    out = np.empty(x.shape, np.uint8)
    if cvec:
        out[..., :cvec] = quantize_u8(np.ascontiguousarray(x[..., :cvec]), inv_s, 128, 2)
    if cvec < Cin:
        out[..., cvec:] = quantize_u8(np.ascontiguousarray(x[..., cvec:]), inv_s, 128, 1)
    return out


def conv_int8_centered_acc(inQ, wq, KH, KW, Cout, stride, pad):
    """A = sum over in-image taps of (u8 - 128) * wq, int32 [N, OH, OW, Cout]."""
    N, H, W, Cin = inQ.shape
    OH, OW = out_hw(H, W, KH, KW, stride, pad)
    acc = np.empty((N, OH, OW, Cout), np.int32)
    lib().oracle_conv_int8_centered_acc(np.ascontiguousarray(inQ), N, H, W, Cin,
                                        np.ascontiguousarray(wq), KH, KW, Cout, stride, pad,
                                        OH, OW, acc)
    return acc


def wino_int8_epilogue(acc, s_in, ws, b, act):
    M = acc.size // acc.shape[-1]
    Cout = acc.shape[-1]
    out = np.empty(acc.shape, np.float32)
    lib().oracle_wino_int8_epilogue(np.ascontiguousarray(acc, np.int32), M, Cout,
                                    np.float32(s_in), np.ascontiguousarray(ws, np.float32),
                                    ptr(b), out, act)
    return out


def conv2d_int8_q(q, s_in, wq, ws, b, KH, KW, Cout, stride, pad, act, rule=0):
    """(out s8 [N,OH,OW,Cout], s_out): the int8-in / int8-out convolution
    (oracle_conv2d_int8_q) of s8 activations q with per-tensor scale s_in."""
    N, H, W, Cin = q.shape
    OH, OW = out_hw(H, W, KH, KW, stride, pad)
    out = np.zeros((N, max(OH, 0), max(OW, 0), Cout), np.int8)
    so = C.c_float(0.0)
    lib().oracle_conv2d_int8_q(np.ascontiguousarray(q, np.int8), np.float32(s_in), N, H, W, Cin,
                               np.ascontiguousarray(wq, np.int8),
                               np.ascontiguousarray(ws, np.float32), ptr(b), KH, KW, Cout, stride,
                               pad, out, C.byref(so), act, rule)
    return out, np.float32(so.value)


def conv2d_int8_route(H, W, Cin, KH, KW, Cout, stride, pad):
    return lib().oracle_conv2d_int8_route(H, W, Cin, KH, KW, Cout, stride, pad)


def conv2d_route(N, H, W, Cin, KH, KW, Cout, stride, pad, groups):
    return lib().oracle_conv2d_route(N, H, W, Cin, KH, KW, Cout, stride, pad, groups)


def fold_bn(w, b, Cout, groups, mean, var, gamma, beta):
    """Returns folded copies (w', b') per fold_bn_into (src/model.cpp:69-95)."""
    w2 = np.array(w, np.float32, copy=True).ravel()
    has_b = b is not None
    b2 = np.array(b if has_b else np.zeros(Cout), np.float32, copy=True)
    lib().oracle_fold_bn(w2, b2, int(has_b), Cout, w2.size, groups, mean, var, gamma, beta)
    return w2, b2
