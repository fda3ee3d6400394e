"""ctypes binding of libsdu.so (the C ABI in include/sdu.h).

Mirrors the reference's Kotlin-side JNI surface (sd/VulkanBench.kt:22-27:
``unetInit / unetForward / unetForward2 / unetSelfTest / unetProfile /
unetRelease``) plus the op-level interface, for Python callers, tests and the
benchmark.  There is no fallback: if the HIP library is missing, loading fails.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libsdu.so")

SDU_OK = 0
SDU_ERR_DEVICE = -1
SDU_ERR_NOT_INIT = -2
SDU_ERR_ARG = -3
SDU_ERR_WEIGHT = -4
SDU_ERR_IO = -5
SDU_ERR_OOM = -6
SDU_ERR_HIP = -7

SDU_F16 = 1
SDU_F32 = 2
SDU_INIT_RANDOM_AFFINE = 0x1
SDU_INIT_NO_WEIGHTS = 0x2
SDU_EPI_GEGLU = 0x1
SDU_EPI_OUT_F32 = 0x2
SDU_EPI_RELU = 0x4
SDU_EPI_QUICK_GELU = 0x8
SDU_ATTN_CAUSAL = 0x1
SDU_ATTN_Q_LOG2 = 0x2

# every symbol include/sdu.h declares
EXPORTS = [
    "sdu_init", "sdu_release", "sdu_last_error", "sdu_synchronize", "sdu_set_weight",
    "sdu_get_weight", "sdu_param_count", "sdu_forward", "sdu_forward_cfg", "sdu_denoise_lcm",
    "sdu_forward_device", "sdu_denoise_lcm_device", "sdu_denoise_lcm_ex", "sdu_selftest", "sdu_selftest_ex", "sdu_time_proj", "sdu_profile", "sdu_profile_ops",
    "sdu_tensor_alloc", "sdu_tensor_free", "sdu_tensor_upload", "sdu_tensor_download",
    "sdu_tensor_device_ptr", "sdu_tensor_bytes", "sdu_groupnorm", "sdu_groupnorm_noalloc", "sdu_layernorm", "sdu_matmul",
    "sdu_conv2d", "sdu_conv2d_groupnorm", "sdu_attention", "sdu_attention_ex", "sdu_geglu", "sdu_silu", "sdu_add", "sdu_add_bias",
    "sdu_lcm_step", "sdu_taesd_init", "sdu_taesd_decode", "sdu_taesd_decode_device", "sdu_vae_init",
    "sdu_vae_decode", "sdu_vae_decode_device", "sdu_clip_init",
    "sdu_clip_encode", "sdu_clip_encode_device", "sdu_generate", "sdu_calibrate",
]


class SduError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"sdu error {code}: {msg}")
        self.code = code


class SelftestReport(ctypes.Structure):
    _fields_ = [("relerr_b1", ctypes.c_double), ("relerr_b2", ctypes.c_double * 2),
                ("ctx_sens", ctypes.c_double)]


class Calibration(ctypes.Structure):
    _fields_ = [("mfma_tflops", ctypes.c_double), ("mfma_clock_ghz", ctypes.c_double),
                ("copy_gbs", ctypes.c_double)]


class ProfEntry(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("calls", ctypes.c_int), ("ms", ctypes.c_double),
                ("flops", ctypes.c_double), ("bytes", ctypes.c_double)]


_lib = None

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float
SZ = ctypes.c_size_t


def load(path: str = LIB_PATH):
    """Load libsdu.so and declare signatures.  Raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not built; run __graft_entry__.build() (make -C "
                                f"{_PKG_DIR})")
    lib = ctypes.CDLL(path)
    sig = {
        "sdu_init": ([ctypes.POINTER(P), ctypes.c_char_p, ctypes.c_uint64, I], I),
        "sdu_release": ([P], I),
        "sdu_last_error": ([P], ctypes.c_char_p),
        "sdu_synchronize": ([P], I),
        "sdu_set_weight": ([P, ctypes.c_char_p, P, I64], I),
        "sdu_get_weight": ([P, ctypes.c_char_p, P, I64], I),
        "sdu_param_count": ([P, ctypes.POINTER(I64), ctypes.POINTER(I64)], I),
        "sdu_forward": ([P, P, P, P, I, I, I, I, P], I),
        "sdu_forward_cfg": ([P, P, P, P, P, I, I, I, P], I),
        "sdu_denoise_lcm": ([P, P, P, P, I, I, I, I, F, P, P], I),
        "sdu_forward_device": ([P, P, P, P, I, I, I, I, P], I),
        "sdu_denoise_lcm_device": ([P, P, P, P, I, I, I, I, F, P, P], I),
        "sdu_denoise_lcm_ex": ([P, P, P, P, I, I, I, I, F, I, P, ctypes.c_uint64, P], I),
        "sdu_selftest": ([P, ctypes.c_char_p], ctypes.c_double),
        "sdu_selftest_ex": ([P, ctypes.c_char_p, ctypes.POINTER(SelftestReport)], I),
        "sdu_time_proj": ([I, P], I),
        "sdu_profile": ([P, I, I, I, I, P, I, ctypes.POINTER(I), ctypes.POINTER(ctypes.c_double)], I),
        "sdu_profile_ops": ([P, I, P, I, ctypes.POINTER(I), ctypes.POINTER(ctypes.c_double)], I),
        "sdu_tensor_alloc": ([P, I, I, ctypes.POINTER(I64), ctypes.POINTER(P)], I),
        "sdu_tensor_free": ([P, P], I),
        "sdu_tensor_upload": ([P, P, P, SZ], I),
        "sdu_tensor_download": ([P, P, P, SZ], I),
        "sdu_tensor_device_ptr": ([P], P),
        "sdu_tensor_bytes": ([P], SZ),
        "sdu_groupnorm": ([P, P, P, P, P, P, I, I, I, I, I, F, I], I),
        "sdu_groupnorm_noalloc": ([P, P, P, P, P, P, I, I, I, I, I, F, I], I),
        "sdu_layernorm": ([P, P, P, P, P, I, I, F], I),
        "sdu_matmul": ([P, P, P, P, P, P, P, I, I, I, I, I], I),
        "sdu_conv2d": ([P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I], I),
        "sdu_conv2d_groupnorm": ([P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, F, I], I),
        "sdu_attention": ([P, P, P, P, P, I, I, I, I, I, I, I, I, I, F], I),
        "sdu_attention_ex": ([P, P, P, P, P, I, I, I, I, I, I, I, I, I, F, I], I),
        "sdu_taesd_init": ([P, ctypes.c_char_p, ctypes.c_uint64, I], I),
        "sdu_taesd_decode": ([P, P, I, I, I, P], I),
        "sdu_taesd_decode_device": ([P, P, I, I, I, P], I),
        "sdu_vae_init": ([P, ctypes.c_char_p, ctypes.c_uint64, I], I),
        "sdu_vae_decode": ([P, P, I, I, I, P], I),
        "sdu_vae_decode_device": ([P, P, I, I, I, P], I),
        "sdu_clip_init": ([P, ctypes.c_char_p, ctypes.c_uint64, I], I),
        "sdu_clip_encode": ([P, P, I, P], I),
        "sdu_clip_encode_device": ([P, P, I, P], I),
        "sdu_generate": ([P, P, P, I, I, I, F, I, ctypes.c_uint64, P], I),
        "sdu_calibrate": ([P, I, ctypes.POINTER(Calibration)], I),
        "sdu_geglu": ([P, P, P, I, I], I),
        "sdu_silu": ([P, P, P, I64], I),
        "sdu_add": ([P, P, P, P, I64], I),
        "sdu_add_bias": ([P, P, P, I64, I], I),
        "sdu_lcm_step": ([P, P, P, P, I64, I, I, F], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def time_proj(t: int) -> np.ndarray:
    """sdu_time_proj: the 320-d sinusoid timestep embedding (float32)."""
    out = np.empty(320, np.float32)
    st = load().sdu_time_proj(int(t), _ptr(out))
    if st != SDU_OK:
        raise SduError(st, load().sdu_last_error(None).decode())
    return out


class Tensor:
    """Device tensor owned by an Engine (sdu_tensor_alloc / free)."""

    def __init__(self, eng: "Engine", handle, dtype, shape):
        self.eng, self.h, self.dtype, self.shape = eng, handle, dtype, tuple(shape)

    @property
    def nbytes(self) -> int:
        return int(load().sdu_tensor_bytes(self.h))

    @property
    def ptr(self) -> int:
        return int(load().sdu_tensor_device_ptr(self.h) or 0)

    def numpy(self) -> np.ndarray:
        dt = np.float16 if self.dtype == SDU_F16 else np.float32
        out = np.empty(self.shape, dt)
        self.eng._check(load().sdu_tensor_download(self.eng.h, self.h, _ptr(out), out.nbytes))
        return out

    def free(self):
        if self.h:
            load().sdu_tensor_free(self.eng.h, self.h)
            self.h = None

    def __del__(self):
        try:
            if self.h and self.eng.h:
                self.free()
        except Exception:
            pass


class Engine:
    """One sdu_ctx (unetInit ... unetRelease)."""

    def __init__(self, weights_dir: Optional[str] = None, seed: int = 0, flags: int = 0):
        lib = load()
        h = ctypes.c_void_p()
        st = lib.sdu_init(ctypes.byref(h), weights_dir.encode() if weights_dir else None,
                          ctypes.c_uint64(seed & (2**64 - 1)), flags)
        if st != SDU_OK:
            raise SduError(st, lib.sdu_last_error(None).decode())
        self.h = h

    # -- lifecycle -------------------------------------------------------
    def release(self):
        if self.h:
            load().sdu_release(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.release()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def _check(self, st: int):
        if st != SDU_OK:
            raise SduError(st, load().sdu_last_error(self.h).decode())

    def sync(self):
        self._check(load().sdu_synchronize(self.h))

    # -- weights -----------------------------------------------------------
    def set_weight(self, name: str, value: np.ndarray):
        v = np.ascontiguousarray(value, np.float32)
        self._check(load().sdu_set_weight(self.h, name.encode(), _ptr(v), v.size))

    def get_weight(self, name: str, shape) -> np.ndarray:
        out = np.empty(shape, np.float32)
        self._check(load().sdu_get_weight(self.h, name.encode(), _ptr(out), out.size))
        return out

    def param_count(self):
        n, t = I64(), I64()
        self._check(load().sdu_param_count(self.h, ctypes.byref(n), ctypes.byref(t)))
        return n.value, t.value

    # -- UNet ------------------------------------------------------------
    def forward(self, lat: np.ndarray, temb: np.ndarray, ctx: np.ndarray) -> np.ndarray:
        """unetForward: lat [B,4,H,W], temb [320], ctx [B,L,768] -> eps [B,4,H,W]."""
        lat = np.ascontiguousarray(lat, np.float32)
        temb = np.ascontiguousarray(temb, np.float32)
        ctx = np.ascontiguousarray(ctx, np.float32)
        B, _, H, W = lat.shape
        out = np.empty_like(lat)
        self._check(load().sdu_forward(self.h, _ptr(lat), _ptr(temb), _ptr(ctx), B, H, W,
                                       ctx.shape[1], _ptr(out)))
        return out

    def forward_cfg(self, lat, temb, cond, uncond) -> np.ndarray:
        """unetForward2: lat [4,H,W] shared by both slots -> [2,4,H,W] (cond, uncond)."""
        lat = np.ascontiguousarray(lat, np.float32)
        temb = np.ascontiguousarray(temb, np.float32)
        cond = np.ascontiguousarray(cond, np.float32)
        uncond = np.ascontiguousarray(uncond, np.float32)
        _, H, W = lat.shape
        out = np.empty((2,) + lat.shape, np.float32)
        self._check(load().sdu_forward_cfg(self.h, _ptr(lat), _ptr(temb), _ptr(cond), _ptr(uncond),
                                           H, W, cond.shape[0], _ptr(out)))
        return out

    def denoise_lcm(self, lat, cond, uncond, steps=4, guidance=8.0, noise=None) -> np.ndarray:
        lat = np.ascontiguousarray(lat, np.float32)
        cond = np.ascontiguousarray(cond, np.float32)
        uncond = np.ascontiguousarray(uncond, np.float32)
        _, H, W = lat.shape
        nz = None if noise is None else np.ascontiguousarray(noise, np.float32)
        out = np.empty_like(lat)
        self._check(load().sdu_denoise_lcm(self.h, _ptr(lat), _ptr(cond), _ptr(uncond), H, W,
                                           cond.shape[0], steps, guidance, _ptr(nz), _ptr(out)))
        return out

    def forward_device(self, d_lat: int, d_temb: int, d_ctx: int, B, H, W, L, d_out: int):
        self._check(load().sdu_forward_device(self.h, d_lat, d_temb, d_ctx, B, H, W, L, d_out))

    def denoise_lcm_device(self, d_lat, d_cond, d_uncond, H, W, L, steps, guidance, d_noise, d_out):
        self._check(load().sdu_denoise_lcm_device(self.h, d_lat, d_cond, d_uncond, H, W, L, steps,
                                                  guidance, d_noise, d_out))

    def denoise_lcm_ex(self, d_lat, d_cond, d_uncond, H, W, L, steps, guidance, cfg_steps, d_noise,
                       noise_seed, d_out):
        """d_noise may be None: the noise is then drawn on the device from noise_seed."""
        self._check(load().sdu_denoise_lcm_ex(self.h, d_lat, d_cond, d_uncond, H, W, L, steps, guidance,
                                              cfg_steps, d_noise, noise_seed, d_out))

    def selftest(self, fixture_dir: str) -> float:
        return float(load().sdu_selftest(self.h, fixture_dir.encode()))

    def selftest_report(self, fixture_dir: str) -> dict:
        """sdu_selftest_ex: the B=1, B=2 and context-sensitivity legs."""
        r = SelftestReport()
        self._check(load().sdu_selftest_ex(self.h, fixture_dir.encode(), ctypes.byref(r)))
        return {"relerr_b1": r.relerr_b1, "relerr_b2": (r.relerr_b2[0], r.relerr_b2[1]),
                "ctx_sens": r.ctx_sens}

    def profile(self, B, H, W, L=77):
        arr = (ProfEntry * 128)()
        n, tot = I(), ctypes.c_double()
        self._check(load().sdu_profile(self.h, B, H, W, L, arr, 128, ctypes.byref(n),
                                       ctypes.byref(tot)))
        out = {}
        for i in range(min(n.value, 128)):
            e = arr[i]
            out[e.name.decode()] = dict(calls=e.calls, ms=e.ms, flops=e.flops, bytes=e.bytes)
        return out, tot.value

    def profile_ops(self, enable: bool):
        """sdu_profile_ops: enable=True opens a kernel-timing window over op-level calls;
        enable=False closes it and returns ({name: calls/ms/flops/bytes}, total_ms)."""
        if enable:
            self._check(load().sdu_profile_ops(self.h, 1, None, 0, None, None))
            return None
        arr = (ProfEntry * 256)()
        n, tot = I(), ctypes.c_double()
        self._check(load().sdu_profile_ops(self.h, 0, arr, 256, ctypes.byref(n), ctypes.byref(tot)))
        out = {}
        for i in range(min(n.value, 256)):
            e = arr[i]
            out[e.name.decode()] = dict(calls=e.calls, ms=e.ms, flops=e.flops, bytes=e.bytes)
        return out, tot.value

    def calibrate(self, copy_mib: int = 512) -> dict:
        """sdu_calibrate: measured MFMA ceiling, shader clock under it, streaming-copy GB/s."""
        r = Calibration()
        self._check(load().sdu_calibrate(self.h, copy_mib, ctypes.byref(r)))
        return {"mfma_tflops": r.mfma_tflops, "mfma_clock_ghz": r.mfma_clock_ghz, "copy_gbs": r.copy_gbs}

    # -- tensors and ops -------------------------------------------------
    def tensor(self, shape, dtype=SDU_F16) -> Tensor:
        shp = (I64 * len(shape))(*shape)
        h = ctypes.c_void_p()
        self._check(load().sdu_tensor_alloc(self.h, dtype, len(shape), shp, ctypes.byref(h)))
        return Tensor(self, h, dtype, shape)

    def upload(self, a: np.ndarray, dtype=None) -> Tensor:
        if dtype is None:
            dtype = SDU_F32 if a.dtype == np.float32 else SDU_F16
        a = np.ascontiguousarray(a, np.float16 if dtype == SDU_F16 else np.float32)
        t = self.tensor(a.shape, dtype)
        self._check(load().sdu_tensor_upload(self.h, t.h, _ptr(a), a.nbytes))
        return t

    def groupnorm(self, x, gamma, beta, y, B, HW, C1, C2=0, x2=None, groups=32, eps=1e-5, silu=False):
        self._check(load().sdu_groupnorm(self.h, x.h, x2.h if x2 else None, gamma.h, beta.h, y.h,
                                         B, HW, C1, C2, groups, eps, int(silu)))

    def layernorm(self, x, gamma, beta, y, T, C, eps=1e-5):
        self._check(load().sdu_layernorm(self.h, x.h, gamma.h, beta.h, y.h, T, C, eps))

    def matmul(self, a, w, y, M, N, K, bias=None, residual=None, a2=None, K2=0, flags=0):
        self._check(load().sdu_matmul(self.h, a.h, a2.h if a2 else None, w.h,
                                      bias.h if bias else None, residual.h if residual else None,
                                      y.h, M, N, K, K2, flags))

    def conv2d(self, x, w, y, B, H, W, Ci, Co, ksize=3, stride=1, upsample=False, bias=None,
               temb=None, residual=None, flags=0):
        self._check(load().sdu_conv2d(self.h, x.h, w.h, bias.h if bias else None,
                                      temb.h if temb else None, residual.h if residual else None,
                                      y.h, B, H, W, Ci, Co, ksize, stride, int(upsample), flags))

    def conv2d_groupnorm(self, x, w, y, gamma, beta, gn_y, B, H, W, Ci, Co, bias=None, temb=None,
                         residual=None, groups=32, eps=1e-5, silu=True):
        """3x3 conv whose epilogue keeps the GroupNorm statistics, then GroupNorm(+SiLU)."""
        self._check(load().sdu_conv2d_groupnorm(self.h, x.h, w.h, bias.h if bias else None,
                                                temb.h if temb else None, residual.h if residual else None,
                                                y.h, gamma.h, beta.h, gn_y.h, B, H, W, Ci, Co, groups, eps,
                                                int(silu)))

    def attention(self, q, k, v, o, B, heads, Sq, Sk, d, ldq, ldk, ldv, ldo, scale):
        self._check(load().sdu_attention(self.h, q.h, k.h, v.h, o.h, B, heads, Sq, Sk, d, ldq, ldk,
                                         ldv, ldo, scale))

    def attention_ex(self, q, k, v, o, B, heads, Sq, Sk, d, ldq, ldk, ldv, ldo, scale, flags=0):
        self._check(load().sdu_attention_ex(self.h, q.h, k.h, v.h, o.h, B, heads, Sq, Sk, d, ldq, ldk,
                                            ldv, ldo, scale, flags))

    # -- TAESD decoder, CLIP text encoder, end-to-end image -----------------
    def taesd_init(self, weights_dir: Optional[str] = None, seed: int = 0, flags: int = 0):
        self._check(load().sdu_taesd_init(self.h, weights_dir.encode() if weights_dir else None, seed, flags))

    def taesd_decode(self, lat: np.ndarray) -> np.ndarray:
        lat = np.ascontiguousarray(lat, np.float32)
        B, _, H, W = lat.shape
        out = np.empty((B, 3, 8 * H, 8 * W), np.float32)
        self._check(load().sdu_taesd_decode(self.h, _ptr(lat), B, H, W, _ptr(out)))
        return out

    def taesd_decode_device(self, d_lat: int, B, H, W, d_img: int):
        self._check(load().sdu_taesd_decode_device(self.h, d_lat, B, H, W, d_img))

    def vae_init(self, weights_dir: Optional[str] = None, seed: int = 0, flags: int = 0):
        self._check(load().sdu_vae_init(self.h, weights_dir.encode() if weights_dir else None, seed, flags))

    def vae_decode(self, lat: np.ndarray) -> np.ndarray:
        lat = np.ascontiguousarray(lat, np.float32)
        B, _, H, W = lat.shape
        out = np.empty((B, 3, 8 * H, 8 * W), np.float32)
        self._check(load().sdu_vae_decode(self.h, _ptr(lat), B, H, W, _ptr(out)))
        return out

    def vae_decode_device(self, d_lat: int, B, H, W, d_img: int):
        self._check(load().sdu_vae_decode_device(self.h, d_lat, B, H, W, d_img))

    def clip_init(self, weights_dir: Optional[str] = None, seed: int = 0, flags: int = 0):
        self._check(load().sdu_clip_init(self.h, weights_dir.encode() if weights_dir else None, seed, flags))

    def clip_encode(self, ids: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        B = ids.shape[0]
        out = np.empty((B, 77, 768), np.float32)
        self._check(load().sdu_clip_encode(self.h, _ptr(ids), B, _ptr(out)))
        return out

    def clip_encode_device(self, d_ids: int, B, d_out: int):
        self._check(load().sdu_clip_encode_device(self.h, d_ids, B, d_out))

    def generate(self, cond_ids, uncond_ids, H=64, W=64, steps=4, guidance=8.0, cfg_steps=None,
                 seed=42) -> np.ndarray:
        cond_ids = np.ascontiguousarray(cond_ids, np.int32)
        uncond_ids = np.ascontiguousarray(uncond_ids, np.int32)
        img = np.empty((3, 8 * H, 8 * W), np.float32)
        self._check(load().sdu_generate(self.h, _ptr(cond_ids), _ptr(uncond_ids), H, W, steps, guidance,
                                        steps if cfg_steps is None else cfg_steps, seed, _ptr(img)))
        return img

    def geglu(self, g, y, T, C2):
        self._check(load().sdu_geglu(self.h, g.h, y.h, T, C2))

    def silu(self, x, y, n):
        self._check(load().sdu_silu(self.h, x.h, y.h, n))

    def add(self, a, b, y, n):
        self._check(load().sdu_add(self.h, a.h, b.h, y.h, n))

    def add_bias(self, y, bias, n, C):
        self._check(load().sdu_add_bias(self.h, y.h, bias.h, n, C))

    def lcm_step(self, x, eps2, noise, n, steps, idx, guidance):
        self._check(load().sdu_lcm_step(self.h, x.h, eps2.h, noise.h if noise else None, n, steps,
                                        idx, guidance))


# reference-named aliases (sd/VulkanBench.kt:22-27)
def unet_init(weights_dir: Optional[str] = None, seed: int = 0, flags: int = 0) -> Engine:
    return Engine(weights_dir, seed, flags)
