"""Thin object layer over the C ABI: a device context, q4nx matrices and MoE layers.

Host-array methods take and return NumPy arrays (bf16 as uint16); ``*_dev`` methods
take torch tensors that already live on the GPU and queue work on a stream without
allocating (they are what the benchmark times and what a HIP graph captures).
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import ACT_SITU, ACT_SWIGLU, BUNDLE_B1, BUNDLE_B2, PART_DOWN, PART_GATE_UP, SCORE_SIGMOID, SCORE_SOFTMAX, call, ptr
from .geometry import MoeGeometry


def act_code(gate_beta, value_beta) -> tuple[int, float, float]:
    """SwiGLU when ``gate_beta is None`` (kernels/moe/reference.py:151-171 convention), else SiTU."""
    if gate_beta is None or value_beta is None:
        if (gate_beta is None) != (value_beta is None):
            raise ValueError("gate_beta and value_beta must be provided together")
        return ACT_SWIGLU, 0.0, 0.0
    return ACT_SITU, float(gate_beta), float(value_beta)


def _u16(a, name: str) -> np.ndarray:
    arr = np.ascontiguousarray(a)
    if arr.dtype != np.uint16:
        raise ValueError(f"{name} must be uint16 (bf16 bits), got {arr.dtype}")
    return arr


def _check_dev(t, shape: tuple, dtype_name: str, name: str):
    """A device tensor must have exactly the shape/dtype the kernel indexes (no OOB on the GPU)."""
    if not hasattr(t, "data_ptr") or not getattr(t, "is_cuda", False):
        raise ValueError(f"{name} must be a GPU tensor")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if str(t.dtype).split(".")[-1] != dtype_name:
        raise ValueError(f"{name} must be {dtype_name}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


_HIP_STREAM_LEGACY = 1  # hipStreamLegacy: the null stream, with its implicit ordering


def _stream_ptr(stream) -> int | None:
    """The HIP stream handle for a ``stream`` argument: None selects the context's own
    stream (the library's NULL).  A torch stream whose handle is 0 -- torch's default
    stream, HIP's null stream -- is passed as hipStreamLegacy, since a 0 handle would
    select the context's stream, which is not ordered with torch's work."""
    if stream is None:
        return None
    if hasattr(stream, "cuda_stream"):
        return stream.cuda_stream or _HIP_STREAM_LEGACY
    return int(stream)


class Context:
    """One device context (``rmoe_create``); owns weights and scratch on one GPU."""

    def __init__(self, device: int = 0):
        lib = _lib.load()
        h = C.c_void_p()
        _lib.check(lib.rmoe_create(int(device), C.byref(h)))
        self._h = h
        self.device = int(device)

    @property
    def handle(self):
        return self._h

    @property
    def stream(self) -> int:
        return _lib.load().rmoe_stream(self._h)

    def close(self):
        if self._h is not None and self._h.value:
            _lib.load().rmoe_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        call("rmoe_synchronize", self._h)

    # ------------------------------------------------------------ matrices --
    def upload_matrix(self, packed: bytes | np.ndarray, M: int, K: int, fmt: str = "q4nx") -> "Matrix":
        """Upload an [M, K] matrix: ``fmt`` "q4nx" (quant/q4nx.py pack_gemv bytes), "bfp16"
        (quant/bfp16.py pack_bfp16_gemv, 9 bits per weight) or "q4k" (a row-major llama.cpp
        Q4_K tensor, converted to q4nx on the device as quant/gguf_q4k.py:228-233 does)."""
        buf = (np.frombuffer(packed, dtype=np.uint8) if isinstance(packed, (bytes, bytearray))
               else np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1))
        h = C.c_int()
        if fmt == "q4nx":
            call("rmoe_matrix_upload", self._h, ptr(buf), buf.size, int(M), int(K), C.byref(h))
        elif fmt == "bfp16":
            call("rmoe_matrix_upload_bfp16", self._h, ptr(buf), buf.size, int(M), int(K), C.byref(h))
        elif fmt == "q4k":
            call("rmoe_matrix_upload_q4k", self._h, ptr(buf), buf.size, int(M), int(K), C.byref(h))
            fmt = "q4nx"
        else:
            raise ValueError(f"unknown matrix format {fmt!r} (expected 'q4nx', 'bfp16' or 'q4k')")
        return Matrix(self, h.value, M, K, fmt)

    def quantize_matrix(self, w_dev, M: int, K: int, stream=None) -> "Matrix":
        """Quantize an fp32 torch tensor [M, K] on the device (bit-exact quant/q4nx.py:127-200)."""
        _check_dev(w_dev, (M, K), "float32", "w")
        h = C.c_int()
        call("rmoe_matrix_quantize_dev", self._h, ptr(w_dev), int(M), int(K), C.byref(h), _stream_ptr(stream))
        return Matrix(self, h.value, M, K)

    # ------------------------------------------------------------ layers --
    def create_layer(self, layer: int, geom: MoeGeometry) -> "MoeLayer":
        call("rmoe_layer_create", self._h, int(layer), geom.hidden, geom.inter, geom.n_routed, geom.n_shared, geom.top_k)
        return MoeLayer(self, int(layer), geom)

    def create_layer_d(self, layer: int, geom: MoeGeometry) -> "MoeLayer":
        """A layer in the reference's weights-d layout (npu/backend.py:624-700): moe_b1 q4nx
        gate/up of the routed experts, moe_b2 bfp16 down of routed + shared experts."""
        if geom.n_shared != 1:
            raise ValueError("a weights-d layer has exactly one shared expert (moe_b2's last expert)")
        call("rmoe_layer_create_d", self._h, int(layer), geom.hidden, geom.inter, geom.n_routed, geom.top_k)
        return MoeLayer(self, int(layer), geom, d_layout=True)

    # ------------------------------------------------------- decode stack --
    @staticmethod
    def _layer_ids(layers) -> np.ndarray:
        ids = np.ascontiguousarray([l.layer if isinstance(l, MoeLayer) else int(l) for l in layers], dtype=np.int32)
        if ids.size < 1:
            raise ValueError("a decode stack needs at least one layer")
        return ids

    def reserve_decode_stack(self, layers):
        """Size the hand-off buffers of the persistent decode kernel for these layers."""
        ids = self._layer_ids(layers)
        call("rmoe_reserve_decode_stack", self._h, ptr(ids), ids.size)

    def set_stack_wait_limit(self, polls: int = 0):
        """Polls (about a microsecond each) after which a wait of the persistent decode
        kernel gives up; 0 restores the default (about two seconds).  The next synchronous
        call then raises RmoeError naming the workgroup, layer and hand-off that gave up."""
        call("rmoe_set_stack_wait_limit", self._h, int(polls))

    def decode_stack(self, layers, x, residual: bool = True, gate_beta=None, value_beta=None):
        """One token through every layer in ``layers`` (one persistent launch).
        Returns (out u16[H], top_ids int32[L, k], weights f32[L, k])."""
        ids = self._layer_ids(layers)
        lyr0 = layers[0] if isinstance(layers[0], MoeLayer) else None
        xa = _u16(x, "x").reshape(-1)
        k = lyr0.geom.top_k if lyr0 else None
        if k is None:
            raise ValueError("decode_stack takes MoeLayer objects")
        act, gb, vb = act_code(gate_beta, value_beta)
        out = np.empty(xa.size, np.uint16)
        top = np.empty((ids.size, k), np.int32)
        w = np.empty((ids.size, k), np.float32)
        call("rmoe_moe_decode_stack", self._h, ptr(ids), ids.size, ptr(xa), ptr(out), int(bool(residual)), act, gb, vb,
             ptr(top), ptr(w))
        return out, top, w

    def decode_stack_dev(self, layers, x_dev, out_dev, residual: bool = True, gate_beta=None, value_beta=None,
                         ids_dev=None, wts_dev=None, stream=None):
        """Device-pointer form of ``decode_stack`` (no allocation; capturable in a HIP graph).
        x/out: int16 (bf16 bits) [H]; ids_dev/wts_dev (optional): int32/float32 [L, k].
        Every tensor is checked against the shapes the kernel indexes before the launch."""
        ids = self._layer_ids(layers)
        if not isinstance(layers[0], MoeLayer):
            raise ValueError("decode_stack_dev takes MoeLayer objects (their geometry sizes the tensors)")
        g = layers[0].geom
        _check_dev(x_dev, (g.hidden,), "int16", "x")
        _check_dev(out_dev, (g.hidden,), "int16", "out")
        if ids_dev is not None:
            _check_dev(ids_dev, (ids.size, g.top_k), "int32", "ids")
        if wts_dev is not None:
            _check_dev(wts_dev, (ids.size, g.top_k), "float32", "wts")
        act, gb, vb = act_code(gate_beta, value_beta)
        call("rmoe_moe_decode_stack_dev", self._h, ptr(ids), ids.size, ptr(x_dev), ptr(out_dev), int(bool(residual)),
             act, gb, vb, ptr(ids_dev), ptr(wts_dev), _stream_ptr(stream))

    def dispatch(self, top_ids, n_experts: int) -> tuple[np.ndarray, np.ndarray]:
        ids = np.ascontiguousarray(top_ids, dtype=np.int32)
        if ids.ndim != 2:
            raise ValueError("top_ids must have shape [tokens, routes]")
        order = np.empty(ids.size, dtype=np.int32)
        offsets = np.empty(n_experts + 1, dtype=np.int32)
        call("rmoe_dispatch", self._h, ptr(ids), ids.shape[0], ids.shape[1], int(n_experts), ptr(order), ptr(offsets))
        return order, offsets


class Matrix:
    """A q4nx or bfp16 matrix resident on the device (tile layout of its format)."""

    _BITS = {"q4nx": 5, "bfp16": 9}

    def __init__(self, ctx: Context, handle: int, M: int, K: int, fmt: str = "q4nx"):
        self.ctx, self.handle, self.M, self.K, self.fmt = ctx, handle, int(M), int(K), fmt

    @property
    def nbytes(self) -> int:
        """Bytes of the matrix in its GEMV byte layout (also its device footprint)."""
        return self.M * self.K * self._BITS[self.fmt] // 8

    def download(self) -> bytes:
        out = np.empty(self.nbytes, dtype=np.uint8)
        call("rmoe_matrix_download", self.ctx.handle, self.handle, ptr(out), out.size)
        return out.tobytes()

    def linear(self, x: np.ndarray) -> np.ndarray:
        """bf16 ``x[..., K_in]`` (K_in <= K, zero padded) -> bf16 ``[..., M]``."""
        xa = _u16(x, "x")
        lead = xa.shape[:-1]
        rows = xa.reshape(-1, xa.shape[-1])
        y = np.empty((rows.shape[0], self.M), dtype=np.uint16)
        if rows.shape[0]:
            call("rmoe_linear", self.ctx.handle, self.handle, ptr(rows), rows.shape[0], rows.shape[1], ptr(y))
        return y.reshape(*lead, self.M)

    def reserve(self, T: int):
        call("rmoe_reserve_linear", self.ctx.handle, self.handle, int(T))

    def linear_dev(self, x_dev, T: int, y_dev, stream=None):
        _check_dev(x_dev, (T, self.K), "int16", "x")
        _check_dev(y_dev, (T, self.M), "int16", "y")
        call("rmoe_linear_dev", self.ctx.handle, self.handle, ptr(x_dev), int(T), ptr(y_dev), _stream_ptr(stream))

    def free(self):
        call("rmoe_matrix_free", self.ctx.handle, self.handle)


class MoeLayer:
    """One MoE layer (experts + router) resident on the device."""

    def __init__(self, ctx: Context, layer: int, geom: MoeGeometry, d_layout: bool = False):
        self.ctx, self.layer, self.geom = ctx, layer, geom
        self.d_layout = bool(d_layout)
        self.has_router = False

    @property
    def gu_expert_bytes(self) -> int:
        """GEMV bytes of one expert's gate/up (q4nx [2I, H])."""
        return self.geom.gu_bytes

    @property
    def dn_expert_bytes(self) -> int:
        """GEMV bytes of one expert's down: q4nx [H, Ipad], or bfp16 [H, Ipad] in a weights-d layer."""
        g = self.geom
        return g.hidden * g.inter_pad * 9 // 8 if self.d_layout else g.dn_bytes

    def upload_d(self, bundle: int, expert0: int, data: bytes | np.ndarray):
        """Experts ``[expert0, expert0 + n)`` of moe_b1 (``bundle`` 1) or moe_b2 (2) of a
        weights-d layer from ``n`` consecutive expert slices of the bundle file."""
        if bundle not in (BUNDLE_B1, BUNDLE_B2):
            raise ValueError(f"bundle must be {BUNDLE_B1} (moe_b1) or {BUNDLE_B2} (moe_b2), got {bundle!r}")
        buf = (np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray, memoryview))
               else np.ascontiguousarray(data, np.uint8).reshape(-1))
        per = self.gu_expert_bytes if bundle == BUNDLE_B1 else self.dn_expert_bytes
        if buf.size % per:
            raise ValueError(f"moe_b{bundle} slice of {buf.size} bytes is not a whole number of {per}-byte experts")
        call("rmoe_layer_upload_d", self.ctx.handle, self.layer, int(bundle), int(expert0), buf.size // per, ptr(buf),
             buf.size)

    def upload_experts(self, gate_up: bytes | np.ndarray, down: bytes | np.ndarray):
        gu = np.frombuffer(gate_up, np.uint8) if isinstance(gate_up, (bytes, bytearray)) else np.ascontiguousarray(gate_up, np.uint8)
        dn = np.frombuffer(down, np.uint8) if isinstance(down, (bytes, bytearray)) else np.ascontiguousarray(down, np.uint8)
        call("rmoe_layer_upload_experts", self.ctx.handle, self.layer, ptr(gu), gu.size, ptr(dn), dn.size)

    _Q4K_PARTS = {"gate": 0, "up": 1, "down": 2}

    def upload_expert_q4k(self, expert: int, part: str, q4k: bytes | np.ndarray):
        """One part ("gate" [I, H], "up" [I, H] or "down" [H, I]) of an expert from a row-major
        llama.cpp Q4_K tensor, converted to q4nx on the device (quant/gguf_q4k.py:160-186,
        228-233: ``q4nx_components(name, outer_index=expert)`` of ffn_{gate,up,down}_exps)."""
        if part not in self._Q4K_PARTS:
            raise ValueError(f"part must be one of {sorted(self._Q4K_PARTS)}, got {part!r}")
        buf = (np.frombuffer(q4k, np.uint8) if isinstance(q4k, (bytes, bytearray))
               else np.ascontiguousarray(q4k, np.uint8).reshape(-1))
        call("rmoe_layer_upload_expert_q4k", self.ctx.handle, self.layer, int(expert), self._Q4K_PARTS[part], ptr(buf),
             buf.size)

    def quantize_expert(self, expert: int, gate_up_dev, down_dev, stream=None):
        g = self.geom
        _check_dev(gate_up_dev, (2 * g.inter, g.hidden), "float32", "gate_up")
        _check_dev(down_dev, (g.hidden, g.inter), "float32", "down")
        call("rmoe_layer_quantize_expert_dev", self.ctx.handle, self.layer, int(expert), ptr(gate_up_dev),
             ptr(down_dev), _stream_ptr(stream))

    def synthesize(self, seed: int, std: float = 0.02, stream=None):
        """Seeded N(0, std) weights for every expert, generated and quantized on the device."""
        call("rmoe_layer_synthesize_dev", self.ctx.handle, self.layer, int(seed) & (2**64 - 1), float(std),
             _stream_ptr(stream))

    def expert_matrix(self, expert: int, part: str) -> "Matrix":
        """A matrix handle viewing one expert's weights in place: ``part`` "gate_up" (q4nx
        ``[2I, H]``, gate rows then up rows) or "down" (``[H, Ipad]``, bfp16 in a weights-d
        layer).  No copy; freeing or re-creating the layer invalidates it."""
        codes = {"gate_up": PART_GATE_UP, "down": PART_DOWN}
        if part not in codes:
            raise ValueError(f"part must be 'gate_up' or 'down', got {part!r}")
        h = C.c_int()
        call("rmoe_layer_expert_matrix", self.ctx.handle, self.layer, int(expert), codes[part], C.byref(h))
        g = self.geom
        if part == "gate_up":
            return Matrix(self.ctx, h.value, 2 * g.inter, g.hidden, "q4nx")
        return Matrix(self.ctx, h.value, g.hidden, g.inter_pad, "bfp16" if self.d_layout else "q4nx")

    def download_expert(self, expert: int) -> tuple[bytes, bytes]:
        """(gate_up, down) GEMV bytes of one expert; gate_up is b"" for the shared expert
        of a weights-d layer, whose gate/up lives outside the layer."""
        no_gu = self.d_layout and int(expert) == self.geom.n_routed
        gu = None if no_gu else np.empty(self.gu_expert_bytes, np.uint8)
        dn = np.empty(self.dn_expert_bytes, np.uint8)
        call("rmoe_layer_download_expert", self.ctx.handle, self.layer, int(expert), ptr(gu), 0 if no_gu else gu.size,
             ptr(dn), dn.size)
        return (b"" if no_gu else gu.tobytes()), dn.tobytes()

    def set_router(self, weight_bf16, bias=None, score: str = "softmax", renormalize: bool = True, scaling: float = 1.0):
        code = {"sigmoid": SCORE_SIGMOID, "softmax": SCORE_SOFTMAX}[score]
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        if b is not None and b.shape != (self.geom.n_routed,):
            raise ValueError(f"router bias must be [{self.geom.n_routed}]")
        if hasattr(weight_bf16, "data_ptr"):
            dt = str(weight_bf16.dtype).split(".")[-1]
            _check_dev(weight_bf16, (self.geom.n_routed, self.geom.hidden), dt if dt in ("bfloat16", "int16") else "bfloat16",
                       "router weight")
            call("rmoe_layer_set_router_dev", self.ctx.handle, self.layer, ptr(weight_bf16), ptr(b), code,
                 int(bool(renormalize)), float(scaling))
        else:
            w = _u16(weight_bf16, "router weight")
            if w.shape != (self.geom.n_routed, self.geom.hidden):
                raise ValueError(f"router weight must be [{self.geom.n_routed}, {self.geom.hidden}]")
            call("rmoe_layer_set_router", self.ctx.handle, self.layer, ptr(w), ptr(b), code, int(bool(renormalize)),
                 float(scaling))
        self.has_router = True

    def reserve(self, max_tokens: int):
        call("rmoe_reserve", self.ctx.handle, self.layer, int(max_tokens))

    def route(self, x: np.ndarray):
        xa = _u16(x, "x").reshape(-1, self.geom.hidden)
        T, k, E = xa.shape[0], self.geom.top_k, self.geom.n_routed
        ids = np.empty((T, k), np.int32)
        wts = np.empty((T, k), np.float32)
        logits = np.empty((T, E), np.float32)
        call("rmoe_route", self.ctx.handle, self.layer, ptr(xa), T, ptr(ids), ptr(wts), ptr(logits))
        return ids, wts, logits

    def moe_experts(self, x, top_ids, top_weights, gate_beta=4.0, value_beta=25.0) -> np.ndarray:
        xa = _u16(x, "x").reshape(-1)
        ids = np.ascontiguousarray(top_ids, dtype=np.int32).reshape(-1)
        w = np.ascontiguousarray(top_weights, dtype=np.float32).reshape(-1)
        if ids.size != w.size:
            raise ValueError("top_ids and top_weights must have the same length")
        act, gb, vb = act_code(gate_beta, value_beta)
        out = np.empty(self.geom.hidden, np.uint16)
        call("rmoe_moe_experts", self.ctx.handle, self.layer, ptr(xa), ptr(ids), ptr(w), ids.size, act, gb, vb, ptr(out))
        return out

    def moe_experts_dev(self, x_dev, ids_dev, wts_dev, out_dev, gate_beta=4.0, value_beta=25.0, stream=None):
        """Device-pointer ``moe_experts`` (no allocation; capturable): x [H] int16 (bf16 bits),
        ids [k] int32, wts [k] float32, out [H] int16."""
        g = self.geom
        _check_dev(x_dev, (g.hidden,), "int16", "x")
        _check_dev(out_dev, (g.hidden,), "int16", "out")
        k = int(ids_dev.shape[0]) if hasattr(ids_dev, "shape") and len(ids_dev.shape) == 1 else -1
        _check_dev(ids_dev, (k,), "int32", "ids")
        _check_dev(wts_dev, (k,), "float32", "wts")
        act, gb, vb = act_code(gate_beta, value_beta)
        call("rmoe_moe_experts_dev", self.ctx.handle, self.layer, ptr(x_dev), ptr(ids_dev), ptr(wts_dev), k, act, gb,
             vb, ptr(out_dev), _stream_ptr(stream))

    def moe_experts_static_dev(self, x_dev, ids_dev, wts_dev, out_dev, gate_beta=4.0, value_beta=25.0, stream=None):
        """``moe_experts_dev`` on the library's static per-device scratch: allocates nothing
        and needs no ``reserve``; calls overlapping on one GPU race."""
        g = self.geom
        _check_dev(x_dev, (g.hidden,), "int16", "x")
        _check_dev(out_dev, (g.hidden,), "int16", "out")
        k = int(ids_dev.shape[0]) if hasattr(ids_dev, "shape") and len(ids_dev.shape) == 1 else -1
        _check_dev(ids_dev, (k,), "int32", "ids")
        _check_dev(wts_dev, (k,), "float32", "wts")
        act, gb, vb = act_code(gate_beta, value_beta)
        call("rmoe_moe_experts_static_dev", self.ctx.handle, self.layer, ptr(x_dev), ptr(ids_dev), ptr(wts_dev), k,
             act, gb, vb, ptr(out_dev), _stream_ptr(stream))

    def moe_decode(self, x, residual: bool = False, gate_beta=None, value_beta=None):
        """Router + routed + shared + combine for one token; returns (out, top_ids, weights)."""
        xa = _u16(x, "x").reshape(-1)
        act, gb, vb = act_code(gate_beta, value_beta)
        out = np.empty(self.geom.hidden, np.uint16)
        ids = np.empty(self.geom.top_k, np.int32)
        w = np.empty(self.geom.top_k, np.float32)
        call("rmoe_moe_decode", self.ctx.handle, self.layer, ptr(xa), ptr(out), int(bool(residual)), act, gb, vb,
             ptr(ids), ptr(w))
        return out, ids, w

    def moe_decode_dev(self, x_dev, out_dev, residual: bool = False, gate_beta=None, value_beta=None,
                       ids_dev=None, wts_dev=None, stream=None):
        act, gb, vb = act_code(gate_beta, value_beta)
        g = self.geom
        _check_dev(x_dev, (g.hidden,), "int16", "x")
        _check_dev(out_dev, (g.hidden,), "int16", "out")
        if ids_dev is not None:
            _check_dev(ids_dev, (g.top_k,), "int32", "ids")
        if wts_dev is not None:
            _check_dev(wts_dev, (g.top_k,), "float32", "wts")
        call("rmoe_moe_decode_dev", self.ctx.handle, self.layer, ptr(x_dev), ptr(out_dev), int(bool(residual)), act,
             gb, vb, ptr(ids_dev), ptr(wts_dev), _stream_ptr(stream))

    def moe_decode_stage_dev(self, stage: int, x_dev, out_dev=None, residual: bool = False, gate_beta=None,
                             value_beta=None, stream=None):
        """Launch one decode stage (0 router, 1 gate/up + activation, 2 down + combine)."""
        act, gb, vb = act_code(gate_beta, value_beta)
        g = self.geom
        _check_dev(x_dev, (g.hidden,), "int16", "x")
        if out_dev is not None:
            _check_dev(out_dev, (g.hidden,), "int16", "out")
        call("rmoe_moe_decode_stage_dev", self.ctx.handle, self.layer, int(stage), ptr(x_dev), ptr(out_dev),
             int(bool(residual)), act, gb, vb, _stream_ptr(stream))

    def moe_experts_grouped(self, x, top_ids, top_weights, shared_gu, gate_beta=4.0, value_beta=25.0):
        xa = _u16(x, "x")
        T = xa.shape[0]
        ids = np.ascontiguousarray(top_ids, dtype=np.int32)
        w = np.ascontiguousarray(top_weights, dtype=np.float32)
        sgu = _u16(shared_gu, "shared_gu")
        act, gb, vb = act_code(gate_beta, value_beta)
        routed = np.empty((T, self.geom.hidden), np.uint16)
        sdown = np.empty((T, self.geom.hidden), np.uint16)
        call("rmoe_moe_experts_grouped", self.ctx.handle, self.layer, ptr(xa), T, ptr(ids), ptr(w), ptr(sgu), act, gb,
             vb, ptr(routed), ptr(sdown))
        return routed, sdown

    def moe_experts_grouped_dev(self, x_dev, ids_dev, wts_dev, shared_gu_dev, routed_dev, sdown_dev, gate_beta=4.0,
                                value_beta=25.0, stream=None):
        """moe_experts_grouped on device tensors: x int16 [T, H], ids int32 [T, k], wts
        float32 [T, k], shared_gu int16 [T, 2I] -> routed, sdown int16 [T, H], queued on
        `stream` (asynchronous; call reserve(T) first)."""
        g = self.geom
        T = int(x_dev.shape[0]) if hasattr(x_dev, "shape") else -1
        _check_dev(x_dev, (T, g.hidden), "int16", "x")
        _check_dev(ids_dev, (T, g.top_k), "int32", "ids")
        _check_dev(wts_dev, (T, g.top_k), "float32", "wts")
        _check_dev(shared_gu_dev, (T, 2 * g.inter), "int16", "shared_gu")
        _check_dev(routed_dev, (T, g.hidden), "int16", "routed")
        _check_dev(sdown_dev, (T, g.hidden), "int16", "shared_down")
        act, gb, vb = act_code(gate_beta, value_beta)
        call("rmoe_moe_experts_grouped_dev", self.ctx.handle, self.layer, ptr(x_dev), T, ptr(ids_dev), ptr(wts_dev),
             ptr(shared_gu_dev), act, gb, vb, ptr(routed_dev), ptr(sdown_dev), _stream_ptr(stream))

    def moe_prefill_dev(self, x_dev, T: int, out_dev, residual: bool = False, gate_beta=None, value_beta=None,
                        ids_dev=None, wts_dev=None, stream=None):
        act, gb, vb = act_code(gate_beta, value_beta)
        g = self.geom
        _check_dev(x_dev, (T, g.hidden), "int16", "x")
        _check_dev(out_dev, (T, g.hidden), "int16", "out")
        if ids_dev is not None:
            _check_dev(ids_dev, (T, g.top_k), "int32", "ids")
        if wts_dev is not None:
            _check_dev(wts_dev, (T, g.top_k), "float32", "wts")
        call("rmoe_moe_prefill_dev", self.ctx.handle, self.layer, ptr(x_dev), int(T), ptr(out_dev), int(bool(residual)),
             act, gb, vb, ptr(ids_dev), ptr(wts_dev), _stream_ptr(stream))

    def free(self):
        call("rmoe_layer_free", self.ctx.handle, self.layer)
