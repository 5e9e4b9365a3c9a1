"""GpuBackend: the MI355X drop-in for the MoE side of raon-npu's NPU backend.

``RaonModel`` (host/raon.py) and ``Engine`` (serve/engine.py) drive a backend
through the ``Backend`` interface of ``host/backend.py:65-204`` plus the NPU
extras ``moe_experts_grouped``/``preload``/``set_step`` (npu/backend.py:4845,
3265, 2805).  This class keeps those method names, argument meanings, dtypes
and exception types for the q4nx MoE path:

* ``linear`` / ``linear_batch``  -- q4nx bundle GEMV (npu/backend.py:3569-3721)
* ``moe_experts``                -- routed experts of one token (host/backend.py:98-117)
* ``moe_experts_grouped``        -- grouped prefill (npu/backend.py:4845-4979)
* ``moe_prestart_shared`` & co.  -- overlap hooks, no-ops here (results never depend on them)
* ``prefill_shared_precompute`` / ``prefill_grouped_moe`` flags (npu/backend.py:2523-2547)

Weights are registered from the reference's q4nx byte layouts (``pack_gemv``
bundles); the device re-lays them at upload.  The attention-side methods of
the reference ``Backend`` (RDA, MLA) are outside the MoE hot path and raise
``NotImplementedError``.
"""

from __future__ import annotations

import time
from collections import defaultdict
from dataclasses import dataclass

import numpy as np

from .device import Context, Matrix, MoeLayer, act_code
from .geometry import MoeGeometry


def _f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, RNE, NaN -> 0x7FC0 (host/weights.py:104-115): input conversion only."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32)
    out = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        out[nan] = 0x7FC0
    return out


def _bf16_to_f32(u: np.ndarray) -> np.ndarray:
    return (np.asarray(u, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


@dataclass
class _Component:
    """A named projection served by a row slice of a bundle (npu/backend.py:360-392)."""

    bundle: str
    row_start: int
    row_end: int
    orig_k: int


class GpuBackend:
    """MoE hot path of the raon-npu backend on one MI355X (gfx950)."""

    _TIMING_KEYS = ("linear_gpu", "moe_gpu", "moe_grouped_gpu", "moe_host", "route_gpu")

    def __init__(self, device: int = 0, *, activation: str | None = None, weights_dir=None, manifest_path=None,
                 layers=None, top_k: int = 6, context: Context | None = None):
        """``weights_dir``/``manifest_path`` load a weights-d directory as the NpuBackend
        constructor does (npu/backend.py:2404-2412); ``context`` shares an existing device
        context instead of creating one on ``device``."""
        self.ctx = context if context is not None else Context(device)
        self.activation = activation  # "swiglu" forces SwiGLU; None follows the betas
        self._bundles: dict[str, Matrix] = {}
        self._components: dict[str, _Component] = {}
        self._layers: dict[int, MoeLayer] = {}
        self._step_id = 0
        self._bundle_cache: dict[str, tuple[int, int, np.ndarray]] = {}
        self._cached_inputs: dict[str, np.ndarray] = {}
        self.prefill_shared_precompute: bool = True
        self.prefill_grouped_moe: bool = True
        self.timings: dict[str, float] = {}
        self.call_counts: dict[str, int] = defaultdict(int)
        self.reset_timings()
        if weights_dir is not None:
            self.load_weights_d(weights_dir, manifest_path, layers=layers, top_k=top_k)

    # ----------------------------------------------------------- bookkeeping --
    def reset_timings(self) -> None:
        self.timings = {k: 0.0 for k in self._TIMING_KEYS}
        self.call_counts = defaultdict(int)

    def _add_timing(self, key: str, dt: float, count: int = 1) -> None:
        self.timings[key] = self.timings.get(key, 0.0) + dt
        self.call_counts[key] += count

    def set_step(self, step: int) -> None:
        """Token step id for the bundle-reuse rule (npu/backend.py:2805)."""
        self._step_id = int(step)

    def preload(self, num_layers: int | None = None) -> None:
        """Weights are resident from registration on; nothing to stage (npu/backend.py:3265)."""
        return None

    def reset(self) -> None:
        """MoE is stateless; clears only the per-step bundle cache."""
        self._bundle_cache.clear()
        self._cached_inputs.clear()

    # ---------------------------------------------------------- registration --
    _FORMATS = {"q4nx_gemv": "q4nx", "bfp16_gemv": "bfp16", "gguf_q4_k": "q4k"}

    def register_bundle(self, bundle: str, packed: bytes | np.ndarray, M: int, K: int, fmt: str = "q4nx_gemv") -> None:
        """Upload one dense bundle: an [M, K] matrix in the reference's ``BundleMeta.fmt``
        (npu/backend.py:104-117): "q4nx_gemv" (quant/q4nx.py pack_gemv) or "bfp16_gemv"
        (quant/bfp16.py pack_bfp16_gemv); or "gguf_q4_k", a row-major llama.cpp Q4_K tensor
        that the device converts to q4nx (quant/gguf_q4k.py:160-186, 228-233), for a
        projection exported straight from the GGUF (e.g. dense_gu or an lm_head)."""
        if fmt not in self._FORMATS:
            raise ValueError(f"Unknown bundle format for {bundle}: {fmt!r}")
        self._bundles[bundle] = self.ctx.upload_matrix(packed, M, K, fmt=self._FORMATS[fmt])

    def register_view(self, bundle: str, matrix: Matrix) -> None:
        """Serve an existing device matrix (e.g. ``MoeLayer.expert_matrix``, a view of an
        expert's tiles) under the bundle name ``bundle``."""
        self._bundles[bundle] = matrix

    def register_component(self, name: str, bundle: str, row_start: int, row_end: int, orig_k: int | None = None) -> None:
        """Serve weight ``name`` as rows ``[row_start, row_end)`` of ``bundle``."""
        mat = self._bundles[bundle]
        if not 0 <= row_start < row_end <= mat.M:
            raise ValueError(f"rows [{row_start}, {row_end}) outside bundle {bundle!r} with {mat.M} rows")
        self._components[name] = _Component(bundle, row_start, row_end, orig_k or mat.K)

    def register_moe_layer(self, layer: int, geom: MoeGeometry, gate_up: bytes | np.ndarray, down: bytes | np.ndarray,
                           router_weight: np.ndarray | None = None, router_bias: np.ndarray | None = None,
                           score: str = "softmax", renormalize: bool = True, scaling: float = 1.0) -> MoeLayer:
        """Upload one layer's expert bundles (kernels/moe/pack.py geometry) and optional router."""
        lyr = self.ctx.create_layer(layer, geom)
        lyr.upload_experts(gate_up, down)
        if router_weight is not None:
            lyr.set_router(router_weight, router_bias, score, renormalize, scaling)
        self._layers[int(layer)] = lyr
        self._register_shared(lyr)
        return lyr

    def _shared_prefix(self, layer: int) -> str:
        return f"model.layers.{int(layer)}.moe.shared_experts"

    def _register_shared(self, lyr: MoeLayer) -> None:
        """Serve the shared expert of a q4nx layer (expert ``n_routed`` of its bundles,
        kernels/moe/pack.py:40-44) under the names ``RaonModel`` asks ``linear`` /
        ``linear_batch`` for (host/raon.py:1314-1323, 1570-1577): gate = rows [0, I) and
        up = rows [I, 2I) of the expert's gate/up matrix, down = its ``[H, Ipad]`` matrix
        with input width I.  The matrices are views of the layer's own tiles (no second
        upload); gate and up share one bundle, so the bundle-reuse rule computes both rows
        in one launch (npu/backend.py:3652-3663)."""
        g = lyr.geom
        if not g.n_shared:
            return
        pfx, d = self._shared_prefix(lyr.layer), f"L{lyr.layer:02d}"
        e = g.shared_id
        self.register_view(f"{d}/shared_gate_up", lyr.expert_matrix(e, "gate_up"))
        self.register_view(f"{d}/shared_down", lyr.expert_matrix(e, "down"))
        self.register_component(f"{pfx}.gate_proj.weight", f"{d}/shared_gate_up", 0, g.inter)
        self.register_component(f"{pfx}.up_proj.weight", f"{d}/shared_gate_up", g.inter, 2 * g.inter)
        self.register_component(f"{pfx}.down_proj.weight", f"{d}/shared_down", 0, g.hidden, orig_k=g.inter)

    def register_moe_layer_q4k(self, layer: int, geom: MoeGeometry, gate_exps, up_exps, down_exps,
                               router_weight: np.ndarray | None = None, router_bias: np.ndarray | None = None,
                               score: str = "softmax", renormalize: bool = True, scaling: float = 1.0) -> MoeLayer:
        """A layer's experts straight from GGUF Q4_K tensors (``ffn_gate_exps``, ``ffn_up_exps``
        [E, I, H] and ``ffn_down_exps`` [E, H, I], each the row-major bytes of all E experts
        back to back, E = n_routed + n_shared); the device converts every expert part to q4nx
        (quant/gguf_q4k.py:160-186, 228-233).  Requires H % 256 == 0 and I % 256 == 0."""
        g = geom
        lyr = self.ctx.create_layer(layer, g)
        parts = {"gate": (gate_exps, g.inter, g.hidden), "up": (up_exps, g.inter, g.hidden),
                 "down": (down_exps, g.hidden, g.inter)}
        for part, (raw, M, K) in parts.items():
            buf = (np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray))
                   else np.ascontiguousarray(raw, np.uint8).reshape(-1))
            per = M * (K // 256) * 144
            if K % 256 or buf.size != per * g.n_experts:
                raise ValueError(f"{part}_exps: expected {g.n_experts} Q4_K experts of [{M}, {K}] "
                                 f"({per * g.n_experts} bytes), got {buf.size} bytes")
            for e in range(g.n_experts):
                lyr.upload_expert_q4k(e, part, buf[e * per:(e + 1) * per])
        if router_weight is not None:
            lyr.set_router(router_weight, router_bias, score, renormalize, scaling)
        self._layers[int(layer)] = lyr
        self._register_shared(lyr)
        return lyr

    def register_moe_layer_d(self, layer: int, geom: MoeGeometry, moe_b1: bytes | np.ndarray, moe_b2: bytes | np.ndarray,
                             shared_gu: bytes | np.ndarray | None = None, router_weight: np.ndarray | None = None,
                             router_bias: np.ndarray | None = None, score: str = "sigmoid", renormalize: bool = True,
                             scaling: float = 1.0) -> MoeLayer:
        """A layer from in-memory weights-d bundles (npu/backend.py:624-700): ``moe_b1``
        (q4nx_gemv_bundle, ``n_routed`` experts ``[2I, H]``), ``moe_b2`` (bfp16_gemv_bundle,
        ``n_routed + 1`` experts ``[H, Ipad]``, the last the shared down) and optionally
        ``shared_gu`` (bfp16 ``[2I, H]``).  The shared expert's gate/up/down are registered as
        the components ``model.layers.{layer}.moe.shared_experts.{gate,up,down}_proj.weight``,
        served by ``linear`` as ``RaonModel._moe_token`` calls them (host/raon.py:1314-1324)."""
        g = geom
        lyr = self.ctx.create_layer_d(layer, g)
        try:
            b1 = np.frombuffer(moe_b1, np.uint8) if isinstance(moe_b1, (bytes, bytearray)) else np.ascontiguousarray(moe_b1, np.uint8).reshape(-1)
            b2 = np.frombuffer(moe_b2, np.uint8) if isinstance(moe_b2, (bytes, bytearray)) else np.ascontiguousarray(moe_b2, np.uint8).reshape(-1)
            if b1.size != g.n_routed * lyr.gu_expert_bytes:
                raise ValueError(f"moe_b1 has {b1.size} bytes, expected {g.n_routed} x {lyr.gu_expert_bytes}")
            if b2.size != (g.n_routed + 1) * lyr.dn_expert_bytes:
                raise ValueError(f"moe_b2 has {b2.size} bytes, expected {g.n_routed + 1} x {lyr.dn_expert_bytes}")
            lyr.upload_d(1, 0, b1)
            lyr.upload_d(2, 0, b2)
        except BaseException:
            lyr.free()
            raise
        if router_weight is not None:
            lyr.set_router(router_weight, router_bias, score, renormalize, scaling)
        self._layers[int(layer)] = lyr
        pfx, d = f"model.layers.{int(layer)}.moe.shared_experts", f"L{int(layer):02d}"
        if shared_gu is not None:
            self.register_bundle(f"{d}/shared_gu", shared_gu, 2 * g.inter, g.hidden, fmt="bfp16_gemv")
            self.register_component(f"{pfx}.gate_proj.weight", f"{d}/shared_gu", 0, g.inter)
            self.register_component(f"{pfx}.up_proj.weight", f"{d}/shared_gu", g.inter, 2 * g.inter)
        # the shared down is moe_b2's last expert (npu/backend.py:4068-4107): a view, no copy
        self.register_view(f"{d}/shared_down", lyr.expert_matrix(g.n_routed, "down"))
        self.register_component(f"{pfx}.down_proj.weight", f"{d}/shared_down", 0, g.hidden, orig_k=g.inter)
        return lyr

    def load_weights_d(self, weights_dir, manifest_path=None, **kw) -> dict:
        """Validate a weights-d directory's manifest (npu/backend.py:729-929) and load its MoE
        path bundles; see ``weights_d.load_weights_d``."""
        from .weights_d import load_weights_d

        return load_weights_d(self, weights_dir, manifest_path, **kw)

    def layer(self, layer: int) -> MoeLayer:
        try:
            return self._layers[int(layer)]
        except KeyError:
            raise ValueError(f"layer {layer} is not an exported MoE layer") from None

    def __contains__(self, name: str) -> bool:
        return name in self._components or name in self._bundles

    # ---------------------------------------------------------------- linear --
    def _resolve(self, name: str) -> tuple[Matrix, _Component]:
        comp = self._components.get(name)
        if comp is None:
            if name in self._bundles:
                m = self._bundles[name]
                return m, _Component(name, 0, m.M, m.K)
            raise KeyError(f"Weight parameter '{name}' not found in GPU bundle map")
        return self._bundles[comp.bundle], comp

    def linear(self, name: str, x: np.ndarray) -> np.ndarray:
        """``y = x @ W^T`` over a q4nx or bfp16 bundle row slice (npu/backend.py:3569-3721).

        bf16 (uint16) input gives bf16 output.  fp32 input is rounded to bf16 for
        the GEMV and the bf16 result is returned as fp32, as the NPU path does.
        Reuse rule: a bundle computed for the same step and the same input object
        is sliced from the cache (npu/backend.py:3652-3663).
        """
        t0 = time.perf_counter()
        is_f32 = x.dtype == np.float32
        xu = _f32_to_bf16(x) if is_f32 else np.asarray(x, dtype=np.uint16)
        mat, comp = self._resolve(name)
        if xu.shape[-1] != comp.orig_k:
            raise ValueError(f"{name}: input width {xu.shape[-1]} != {comp.orig_k}")
        cached = self._bundle_cache.get(comp.bundle)
        if cached is not None and cached[0] == self._step_id and cached[1] == id(x) and self._cached_inputs.get(comp.bundle) is x:
            y_full = cached[2]
        else:
            y_full = mat.linear(xu)
            self._bundle_cache[comp.bundle] = (self._step_id, id(x), y_full)
            self._cached_inputs[comp.bundle] = x
        out = y_full[..., comp.row_start : comp.row_end].copy()
        self._add_timing("linear_gpu", time.perf_counter() - t0)
        return _bf16_to_f32(out) if is_f32 else out

    def linear_batch(self, name: str, x: np.ndarray) -> np.ndarray:
        """``[T, K]`` -> ``[T, M]``, byte-identical to stacked ``linear`` (host/backend.py:71-74)."""
        if not isinstance(x, np.ndarray) or x.dtype != np.uint16 or x.ndim != 2:
            # npu/backend.py:3399-3400: only a [T, K] uint16 (bf16 bits) array is accepted
            raise ValueError("linear_batch expects a [T, K] uint16 ndarray")
        mat, comp = self._resolve(name)
        if x.shape[1] != comp.orig_k:
            raise ValueError(f"{name}: input width {x.shape[1]} != {comp.orig_k}")
        t0 = time.perf_counter()
        y = mat.linear(x)[:, comp.row_start : comp.row_end].copy()
        self._add_timing("linear_gpu", time.perf_counter() - t0)
        return y

    # overlap hooks (host/backend.py:119-155): results never depend on them
    def moe_prestart_shared(self, layer: int, x: np.ndarray) -> None:
        return None

    def moe_abort_prestart_shared(self) -> None:
        return None

    def prefetch_linears(self, items) -> None:
        return None

    def linear_start(self, name: str, x: np.ndarray) -> object:
        return (name, x)

    def linear_finish(self, pending: object) -> np.ndarray:
        name, x = pending
        return self.linear(name, x)

    def linear_abort(self, pending: object) -> None:
        return None

    # ------------------------------------------------------------------- MoE --
    def _act(self, gate_beta, value_beta):
        if self.activation == "swiglu":
            return None, None
        return gate_beta, value_beta

    def moe_experts(self, layer: int, x: np.ndarray, top_ids: np.ndarray, top_weights: np.ndarray,
                    gate_beta: float | None = 4.0, value_beta: float | None = 25.0,
                    shared_gu: np.ndarray | None = None) -> np.ndarray:
        """Weighted sum of the routed experts for one token (host/backend.py:466-510).

        Experts are combined in ascending id in fp32 and rounded to bf16 once.
        ``shared_gu`` is validated like npu/backend.py:5046-5055 and otherwise
        ignored: the shared expert is not part of this sum.
        """
        lyr = self.layer(layer)
        if shared_gu is not None:
            if not isinstance(shared_gu, np.ndarray) or shared_gu.dtype != np.uint16 or shared_gu.shape != (2 * lyr.geom.inter,):
                raise ValueError(f"shared_gu must be a [{2 * lyr.geom.inter}] uint16 ndarray")
        xu = _f32_to_bf16(x) if x.dtype == np.float32 else np.asarray(x, dtype=np.uint16)
        t0 = time.perf_counter()
        gb, vb = self._act(gate_beta, value_beta)
        out = lyr.moe_experts(xu.reshape(-1)[: lyr.geom.hidden], np.asarray(top_ids), np.asarray(top_weights, np.float32), gb, vb)
        self._add_timing("moe_gpu", time.perf_counter() - t0)
        return out

    def moe_experts_grouped(self, layer: int, x: np.ndarray, top_ids: np.ndarray, top_weights: np.ndarray,
                            shared_gu: np.ndarray, gate_beta: float | None = 4.0,
                            value_beta: float | None = 25.0) -> tuple[np.ndarray, np.ndarray]:
        """Grouped routed sums and shared down rows for ``T`` tokens (npu/backend.py:4845-4979).

        Validation follows npu/backend.py:4864-4897 with the layer's geometry.
        """
        if not isinstance(layer, (int, np.integer)):
            raise ValueError("layer must be an integer")
        lyr = self.layer(int(layer))
        g = lyr.geom
        if not isinstance(x, np.ndarray) or x.dtype != np.uint16 or x.ndim != 2:
            raise ValueError(f"x must be a [T, {g.hidden}] uint16 ndarray")
        if x.shape[0] < 1 or x.shape[1] != g.hidden:
            raise ValueError(f"x must be a [T, {g.hidden}] uint16 ndarray with T >= 1")
        T = x.shape[0]
        if (not isinstance(top_ids, np.ndarray) or not np.issubdtype(top_ids.dtype, np.integer)
                or top_ids.shape != (T, g.top_k)):
            raise ValueError(f"top_ids must be an integer ndarray with shape [T, {g.top_k}]")
        if np.any(top_ids < 0) or np.any(top_ids >= g.n_routed):
            raise ValueError(f"top_ids values must be in 0..{g.n_routed - 1}")
        s = np.sort(top_ids, axis=1)
        if np.any(s[:, 1:] == s[:, :-1]):
            raise ValueError(f"each token must route to {g.top_k} distinct experts")
        if (not isinstance(top_weights, np.ndarray) or top_weights.dtype != np.float32
                or top_weights.shape != (T, g.top_k)):
            raise ValueError(f"top_weights must be a float32 ndarray with shape [T, {g.top_k}]")
        if (not isinstance(shared_gu, np.ndarray) or shared_gu.dtype != np.uint16
                or shared_gu.shape != (T, 2 * g.inter)):
            raise ValueError(f"shared_gu must be a [T, {2 * g.inter}] uint16 ndarray")
        t0 = time.perf_counter()
        gb, vb = self._act(gate_beta, value_beta)
        routed, sdown = lyr.moe_experts_grouped(x, top_ids, top_weights, shared_gu, gb, vb)
        self._add_timing("moe_grouped_gpu", time.perf_counter() - t0, count=T)
        return routed, sdown

    def route(self, layer: int, x: np.ndarray):
        """Device router for ``[T, H]`` or ``[H]`` tokens -> (top int32, weights f32, logits f32)."""
        t0 = time.perf_counter()
        out = self.layer(layer).route(np.asarray(x, dtype=np.uint16))
        self._add_timing("route_gpu", time.perf_counter() - t0)
        return out

    # ------------------------------------------------ outside the MoE hot path --
    def rda_update(self, *a, **k):
        raise NotImplementedError("RDA recurrence is outside the MoE hot path served by GpuBackend")

    def mla_attend(self, *a, **k):
        raise NotImplementedError("MLA attention is outside the MoE hot path served by GpuBackend")

    def mla_attend_chunk(self, *a, **k):
        raise NotImplementedError("MLA attention is outside the MoE hot path served by GpuBackend")

    def set_rda_state(self, *a, **k):
        raise NotImplementedError("RDA state is outside the MoE hot path served by GpuBackend")

    def get_rda_state(self, *a, **k):
        raise NotImplementedError("RDA state is outside the MoE hot path served by GpuBackend")

    def set_mla_cache(self, *a, **k):
        raise NotImplementedError("MLA cache is outside the MoE hot path served by GpuBackend")

    def get_mla_cache(self, *a, **k):
        raise NotImplementedError("MLA cache is outside the MoE hot path served by GpuBackend")
