"""``Muon`` optimizer, world_size=1 owner path on MI355X (reference: ``dmuon/optim/muon.py``).

Constructor, ``step()`` and ``zero_grad()`` keep the reference's signature and error behaviour
(``muon.py:127-314``, ``:1354-1444``, ``:1918``). The per-parameter Muon math of
``_step_muon_params`` (``muon.py:1582-1747``)::

    buf = mu*buf + g            (first step: buf = g)             muon.py:1683-1691
    ns_in = g + mu*buf          (Nesterov; else buf)               muon.py:1693-1694
    U = NS(ns_in)                                                   muon.py:1704
    W *= 1 - lr*wd  (wd > 0);  W += -lr*0.2*sqrt(max(m, n)) * U     muon.py:1728-1740

runs on the GPU as one C-ABI call per bucket of same-shape parameters
(``dmuon_muon_step_group``): a fused momentum/Nesterov/staging kernel, a norm finalise, and
the fp16 MFMA products of the chosen NS form (``ns_backend``: "gram", the default, or
"direct"), the last product applying the weight update in its epilogue. The momentum buffer is fp32 and lives in
``optimizer.state[id(dp)]["momentum_buffer"]`` shaped ``(rows, cols)`` like the reference's.

Parameters that are not dedicated (and 1-D dedicated ones) get the reference's decoupled AdamW
(``muon.py:1857-1916``): its (step, dtype) buckets, each updated by one fused HIP pass
(``dmuon_adamw_multi``) with the rounding points of the reference's ``torch._foreach`` sequence.
"""
from __future__ import annotations

import logging
import math
import os
from collections import OrderedDict
from typing import Optional, Union

import torch
from torch import Tensor, nn

from dmuon_amd import _C
from dmuon_amd.api import iter_dedicated_states
from dmuon_amd.grad_clip import _clip_ready_muon_grad_norm_
from dmuon_amd.utils import prepare_muon_grads
from dmuon_amd.optim.adamw import fused_adamw_
from dmuon_amd.optim.newton_schulz import (NewtonSchulz, _backend_code, _coeff_array,
                                           _float_dtype_code)

logger = logging.getLogger(__name__)

_MUON_KEYS = ("lr", "momentum", "weight_decay")


def _state_tensor(t, shape: tuple, device: torch.device, dtype: torch.dtype, key: str,
                  name: str) -> Tensor:
    """An optimizer-state tensor in the layout the kernels read: on ``device``, ``dtype``,
    contiguous, shaped ``shape``. State restored by ``load_state_dict`` keeps whatever it was
    saved with (the Muon state is keyed by ``id(dp)``, which torch does not cast): a CPU
    ``map_location``, the reference's grad-dtype momentum (``grad.clone()``), a view. Those are
    converted here, once; a tensor of the wrong size raises instead of reaching a kernel."""
    if not torch.is_tensor(t):
        raise TypeError(f"{name}: optimizer state {key!r} must be a tensor, got {type(t).__name__}")
    numel = math.prod(shape)
    if t.numel() != numel:
        raise ValueError(f"{name}: optimizer state {key!r} has {t.numel()} elements, expected "
                         f"{numel} (shape {tuple(shape)})")
    if t.device != device or t.dtype != dtype or not t.is_contiguous() or tuple(t.shape) != shape:
        t = t.detach().to(device=device, dtype=dtype).reshape(shape).contiguous()
    return t


def _pinned_ptrs(ptrs: list[int], device: torch.device) -> Tensor:
    host = torch.tensor(ptrs, dtype=torch.int64, pin_memory=True)
    return host.to(device, non_blocking=True)


class Muon(torch.optim.Optimizer):
    """Muon for dedicated matrix parameters + AdamW for the rest (``muon.py:127-153``).

    Extra keyword arguments of the reference that concern multi-rank scheduling
    (``replicate_async``, ``group_prepare_ahead``, ``tp_distributed_gram*``,
    ``post_step_prefetch_*``, ``forward_prefetch_depth``, ...) are accepted and have no effect
    at world_size=1. ``workspace_limit_bytes`` bounds the NS scratch of one chunk (a bucket of
    same-shape matrices is processed in chunks that fit, sized to waste little of the last wave
    of tiles; the 24 GiB default holds a whole 4096 x 4096 Llama bucket of 64, or 32 of the
    4096 x 14336 ones, in one chunk -- a small part of MI355X's 288 GB); ``overlap_staging=True`` stages the
    next chunk on a side stream while the current chunk's NS runs, with two such workspaces
    (bit-identical results; off by default: on MI355X the concurrent staging traffic slows the
    MFMA kernels by about as much as it hides). ``single_pass_staging=True`` (the default) keeps
    each parameter's last NS input scale ``1/(||ns_in|| + eps)`` in
    ``state[id(dp)]["ns_scale"]`` and stages the fp16 NS operand with it in the momentum pass;
    the first NS products correct the estimate exactly when it is within a factor of 4 of the
    new scale, and the operand is staged again otherwise (always on a parameter's first step).
    This saves the second pass over the gradient and the momentum buffer; results differ from
    ``single_pass_staging=False`` by the fp16 rounding of that operand. After one eager step a
    step of the Muon groups copies nothing to the device (the kernels' pointer tables are kept
    per chunk until a tensor moves), so a caller may capture it into a graph
    (``torch.cuda.graph``) with gradients written into the same tensors between replays;
    AdamW-routed parameters cannot be captured (host step count).
    """

    def __init__(
        self,
        model: nn.Module,
        lr: float = 0.02,
        momentum: float = 0.95,
        weight_decay: float = 0.0,
        ns_steps: int = 5,
        adamw_lr: float = 1e-3,
        adamw_betas: tuple[float, float] = (0.9, 0.999),
        adamw_weight_decay: float = 0.01,
        adamw_eps: float = 1e-8,
        param_groups: Optional[list[dict]] = None,
        ns_backend: Union[str, NewtonSchulz] = "gram",
        nesterov: bool = True,
        record_step_profile: bool = False,
        workspace_limit_bytes: int = 24 << 30,
        ns_eps: float = 1e-7,
        overlap_staging: bool = False,
        single_pass_staging: bool = True,
        **kwargs,
    ):
        if isinstance(ns_backend, str):
            ns_backend = NewtonSchulz(backend=ns_backend)
        if not isinstance(ns_backend, NewtonSchulz):
            raise TypeError(
                f"ns_backend must be 'gram', 'direct', or a NewtonSchulz instance, "
                f"got {type(ns_backend).__name__}")
        comm_ctx = getattr(model, "_dedicated_comm_ctx", None)
        if comm_ctx is None:
            raise ValueError(
                "Model has no _dedicated_comm_ctx. Call dmuon.dedicate_params() first.")
        graph_env = os.environ.get("DMUON_NS_CUDA_GRAPH")
        if graph_env is not None:
            # the reference's per-shape NS graph cache (ns_graph.py:38-47) has no counterpart:
            # say so instead of ignoring the switch silently
            logger.warning(
                "DMUON_NS_CUDA_GRAPH=%s has no effect in dmuon_amd: each bucket's whole Newton-"
                "Schulz runs as one C call that enqueues its kernel launches (no per-NS Python "
                "launch sequence to capture). To remove the host launch cost, capture "
                "Muon.step itself with torch.cuda.graph after one eager step.", graph_env)
        self.model = model
        self._comm_ctx = comm_ctx
        self._ns = ns_backend
        self._ns_steps = ns_steps
        self._nesterov = bool(nesterov)
        self._ns_eps = float(ns_eps)
        self._record_step_profile = bool(record_step_profile)
        self._workspace_limit = int(workspace_limit_bytes)
        self._workspaces: list = [None, None]
        self._ptr_tables: dict = {}
        self._captured_tables: dict = {}      # tables a graph capture has read (kept alive)
        self._overlap_staging = bool(overlap_staging)
        self._single_pass = bool(single_pass_staging)
        self._side_streams: dict = {}
        self._last_step_profile: dict = {}
        self._optimizer_step_index = 0

        self._all_dedicated_params = []
        for st in iter_dedicated_states(model):
            for dp in st.group.params:
                self._all_dedicated_params.append(dp)
        self._dedicated_params = [dp for dp in self._all_dedicated_params if dp.is_owner]

        # Non-dedicated params: FSDP2-managed (if any) or registered through replicate().
        self._fsdp_params: list[nn.Parameter] = []
        fsdp_hit = False
        for module in model.modules():
            fsdp_state = getattr(module, "_get_fsdp_state", lambda: None)()
            if fsdp_state is not None and getattr(fsdp_state, "_fsdp_param_group", None) is not None:
                for fp in fsdp_state._fsdp_param_group.fsdp_params:
                    self._fsdp_params.append(fp.sharded_param)
                fsdp_hit = True
        rep = getattr(model, "_replicated_group", None)
        if rep is not None:
            self._fsdp_params.extend(rep.params)
        non_dedicated_exists = any(
            not hasattr(p, "_dedicated_owner_rank") and p.requires_grad for p in model.parameters())
        if self._all_dedicated_params and non_dedicated_exists and not (fsdp_hit or rep is not None):
            raise RuntimeError(
                "dmuon.Muon: model has non-dedicated parameters but neither "
                "fully_shard nor dmuon.replicate was called. Those parameters "
                "would not be synced across ranks nor updated. Call one of "
                "fully_shard() or dmuon.replicate(model, mesh=...) before "
                "constructing Muon.")

        self._dp_by_param = {id(dp.param): dp for dp in self._dedicated_params}
        groups = self._build_groups(param_groups, lr, momentum, weight_decay, adamw_lr,
                                    adamw_betas, adamw_weight_decay, adamw_eps)
        defaults = dict(lr=lr, momentum=momentum, weight_decay=weight_decay)
        super().__init__(groups, defaults)
        # Muon-routed dedicated params -> their group (the gradients clip_grad_norm_ sees)
        self._dp_to_muon_group_idx: dict[int, int] = {}
        for gi, g in enumerate(self.param_groups):
            if g.get("use_muon", False):
                for p in g["params"]:
                    dp = self._dp_by_param.get(id(p))
                    if dp is not None:
                        self._dp_to_muon_group_idx[id(dp)] = gi
        self._grads_ready = False
        self._last_muon_grad_clip_stats = None

    # ------------------------------------------------------------------ groups
    def _build_groups(self, param_groups, lr, momentum, wd, adamw_lr, betas, adamw_wd, eps):
        """Lowers user groups into Muon (2-D+ dedicated) and AdamW subgroups."""
        muon_ids = {id(dp.param) for dp in self._dedicated_params if dp.param.dim() >= 2}
        adamw_pool = [dp.param for dp in self._dedicated_params if dp.param.dim() < 2]
        adamw_pool += self._fsdp_params
        user = param_groups if param_groups is not None else [
            {"params": [dp.param for dp in self._dedicated_params] + self._fsdp_params}]
        out = []
        seen: set[int] = set()
        for ug in user:
            params = list(ug["params"])
            muon_p = [p for p in params if id(p) in muon_ids and id(p) not in seen]
            adam_p = [p for p in params if id(p) not in muon_ids and id(p) not in seen
                      and p.requires_grad]
            seen.update(id(p) for p in params)
            if muon_p:
                out.append({"params": muon_p, "use_muon": True,
                            "lr": ug.get("lr", lr), "momentum": ug.get("momentum", momentum),
                            "weight_decay": ug.get("weight_decay", wd)})
            if adam_p:
                out.append({"params": adam_p, "use_muon": False,
                            "lr": ug.get("adamw_lr", adamw_lr),
                            "betas": tuple(ug.get("adamw_betas", betas)),
                            "weight_decay": ug.get("adamw_weight_decay", adamw_wd),
                            "eps": ug.get("adamw_eps", eps)})
        missing = [p for p in adamw_pool if id(p) not in seen and p.requires_grad]
        if missing:
            out.append({"params": missing, "use_muon": False, "lr": adamw_lr,
                        "betas": tuple(betas), "weight_decay": adamw_wd, "eps": eps})
        if not out:
            out.append({"params": [], "use_muon": True, "lr": lr, "momentum": momentum,
                        "weight_decay": wd})
        return out

    # ------------------------------------------------------------------ clipping
    def _ensure_grads_ready(self, *, coalesce_wait: bool = False) -> None:
        """``muon.py:1311-1321``: make the owned reduced gradients available, once per step."""
        if self._grads_ready:
            return
        prepare_muon_grads(self.model)
        self._grads_ready = True

    @torch.no_grad()
    def clip_grad_norm_(self, max_norm: Optional[float], *, norm_type: Optional[float] = None,
                        error_if_nonfinite: Optional[bool] = None,
                        foreach: Optional[bool] = None, strategy: Optional[object] = None):
        """Clip the dedicated Muon gradients only (``muon.py:1323-1351``); AdamW-routed
        gradients are left to ``torch.nn.utils.clip_grad_norm_``."""
        self._ensure_grads_ready()
        return _clip_ready_muon_grad_norm_(
            self, max_norm, norm_type=2.0 if norm_type is None else norm_type,
            error_if_nonfinite=False if error_if_nonfinite is None else error_if_nonfinite,
            foreach=foreach, strategy="global_norm" if strategy is None else strategy)

    @property
    def last_muon_grad_clip_stats(self):
        return self._last_muon_grad_clip_stats

    # ------------------------------------------------------------------ step
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        ev = None
        if self._record_step_profile:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        count = numel = 0
        for group in self.param_groups:
            if group.get("use_muon", False):
                c, n = self._step_muon_group(group)
                count += c
                numel += n
        if ev is not None:
            ev[1].record()
        for group in self.param_groups:
            if not group.get("use_muon", False):
                self._step_adamw_group(group)
        if ev is not None:
            self._last_step_profile = {"_events": ev, "ns_matrix_count": count,
                                       "ns_input_numel": numel}
        self._optimizer_step_index += 1
        self._grads_ready = False
        return loss

    def consume_last_step_profile(self) -> dict:
        """``muon.py:1287-1309``: timings of the last step (synchronises on its events)."""
        prof = dict(self._last_step_profile)
        ev = prof.pop("_events", None)
        if ev is not None:
            ev[1].synchronize()
            prof["ns_compute_ms"] = ev[0].elapsed_time(ev[1])
        self._last_step_profile = {}
        return prof

    def _buckets(self, group) -> "OrderedDict[tuple, list]":
        """Owned params with a gradient, grouped by their oriented NS shape (m, n) =
        (min, max) of (rows, cols) and the dtypes the kernels specialise on: a matrix and its
        transpose share every NS product. Each bucket lists (dp, grad, (rows, cols)), the
        params stored m x n first and the transposed (n x m) ones after them, which is the
        order the group entry points take (their last ``n_transposed`` members)."""
        buckets: OrderedDict[tuple, list] = OrderedDict()
        for p in group["params"]:
            dp = self._dp_by_param.get(id(p))
            if dp is None:
                continue
            g = dp.current_grad()
            if g is None:
                continue
            st = self.state[id(dp)]
            first = "momentum_buffer" not in st
            rows = p.shape[0]
            cols = p.numel() // rows
            pub = dp.publish_target()
            key = (min(rows, cols), max(rows, cols), g.dtype, dp._owned_data.dtype,
                   None if pub is None else pub.dtype, g.device, first)
            buckets.setdefault(key, []).append((dp, g, (rows, cols)))
        for items in buckets.values():
            items.sort(key=lambda it: it[2][0] > it[2][1])   # stable: m x n first
        return buckets

    def _step_muon_group(self, group) -> tuple[int, int]:
        """One Muon group: its same-shape buckets, each split into chunks that fit a workspace.

        Each chunk is staged (momentum, norm, NS operands: bandwidth-bound) and then applied
        (NS products + fused update: MFMA-bound). With ``overlap_staging`` the chunks run as a
        two-slot pipeline: chunk k+1 is staged on a side stream into the other workspace while
        chunk k's NS runs on the current stream. Events order every hand-over; the results are
        bit-identical to the one-stream sequence.
        """
        lr, mu, wd = float(group["lr"]), float(group["momentum"]), float(group["weight_decay"])
        coeffs, T = _coeff_array(self._ns.resolved_coefficients())
        backend = _backend_code(self._ns.backend)
        rst, n_rst = _C.restart_array(self._ns.restart_codes())
        chunks = []
        count = numel = 0
        for (rows, cols, gdt, wdt, pdt, dev, first), items in self._buckets(group).items():
            _require_cuda(dev)
            num_cus = torch.cuda.get_device_properties(dev).multi_processor_count
            s0 = 0
            for size in self._chunk_sizes(rows, cols, len(items), num_cus, backend):
                part = items[s0:s0 + size]
                s0 += size
                n_t = sum(1 for _, _, shape in part if shape[0] != rows)
                for dp, _, shape in part:
                    st = self.state[id(dp)]
                    if "momentum_buffer" not in st:
                        st["momentum_buffer"] = torch.zeros(shape, dtype=torch.float32,
                                                            device=dev)
                    else:
                        st["momentum_buffer"] = _state_tensor(
                            st["momentum_buffer"], shape, dev, torch.float32,
                            "momentum_buffer", dp.param_name)
                    if self._single_pass:
                        sc = st.get("ns_scale")
                        if not torch.is_tensor(sc) or sc.numel() != 1:
                            # no usable kept scale: 0 stages the operand exactly
                            st["ns_scale"] = torch.zeros(1, dtype=torch.float32, device=dev)
                        else:
                            st["ns_scale"] = _state_tensor(sc, (1,), dev, torch.float32,
                                                           "ns_scale", dp.param_name)
                    if not dp._owned_data.is_contiguous():
                        raise RuntimeError(f"{dp.param_name}: Muon needs a contiguous weight")
                tile, _, _, nbytes = _C.plan(rows, cols, len(part), 0, num_cus, backend)
                chunks.append((rows, cols, n_t, dev, first, pdt is not None, part, tile, nbytes))
                count += len(part)
                numel += len(part) * rows * cols
        if not chunks:
            return 0, 0
        dev = chunks[0][3]
        main = torch.cuda.current_stream(dev)
        self._run_pipeline(chunks, dev, main, (lr, mu, wd, coeffs, T, backend, rst, n_rst))
        for c in chunks:
            for dp, _, _ in c[6]:
                dp._reduced_grad = None
        return count, numel

    def _stage_chunk(self, chunk, ws, stream, args) -> None:
        """Momentum, norm and NS operands of one chunk into ``ws``, on ``stream`` (the pointer
        arrays and any contiguous gradient copies are made on that stream too)."""
        rows, cols, n_t, dev, first, _, part, tile, _ = chunk
        _, mu, _, _, _, backend, _, _ = args
        L = len(part)
        with torch.cuda.stream(stream):
            gs = [g if g.is_contiguous() else g.contiguous() for _, g, _ in part]
            ests = ([self.state[id(dp)]["ns_scale"].data_ptr() for dp, _, _ in part]
                    if self._single_pass else [])
            ptrs = self._ptr_table(("stage",) + tuple(id(dp) for dp, _, _ in part),
                                   [t.data_ptr() for t in gs]
                                   + [self.state[id(dp)]["momentum_buffer"].data_ptr()
                                      for dp, _, _ in part] + ests, dev)
            _C.call("dmuon_muon_stage_group", ptrs.data_ptr(), _float_dtype_code(gs[0]),
                    ptrs.data_ptr() + 8 * L,
                    ptrs.data_ptr() + 16 * L if ests else None, rows, cols, L, n_t, mu,
                    int(self._nesterov), int(first), backend, self._ns_eps, ws.data_ptr(),
                    ws.numel(), tile, stream.cuda_stream)

    def _apply_chunk(self, chunk, ws, stream, args) -> None:
        """NS products and the fused weight update of one staged chunk, on ``stream``."""
        rows, cols, n_t, dev, _, has_pub, part, tile, _ = chunk
        lr, _, wd, coeffs, T, backend, rst, n_rst = args
        L = len(part)
        with torch.cuda.stream(stream):
            W = [dp._owned_data for dp, _, _ in part]
            pubs = [dp.publish_target() for dp, _, _ in part] if has_pub else []
            wptrs = self._ptr_table(("apply",) + tuple(id(dp) for dp, _, _ in part),
                                    [t.data_ptr() for t in W] + [t.data_ptr() for t in pubs],
                                    dev)
            # the forward copies (master != parameter) are written by the same epilogue
            _C.call("dmuon_muon_apply_group", wptrs.data_ptr(), _float_dtype_code(W[0]),
                    wptrs.data_ptr() + 8 * L if pubs else None,
                    _float_dtype_code(pubs[0]) if pubs else 0, rows, cols, L, n_t, lr, wd,
                    coeffs, T, backend, rst, n_rst, ws.data_ptr(), ws.numel(), tile,
                    stream.cuda_stream)

    def _ptr_table(self, slot: tuple, ptrs: list, device: torch.device) -> Tensor:
        """The device array of ``ptrs`` (int64 addresses) that a group entry point reads, kept
        per ``slot`` (role and the chunk's parameters) and rebuilt only when an address
        changes: a steady-state step copies nothing to the device, which also lets a caller
        capture it into a graph after one eager step. The array is built on the current
        stream, so a replaced one returns to the allocator in that stream's order. A table
        that a graph capture has used is kept alive for the optimizer's lifetime, so an earlier
        graph still reads valid tables after an eager step with moved tensors rebuilt the
        slot's table (the graph keeps operating on the tensors it was captured with)."""
        key = tuple(ptrs)
        hit = self._ptr_tables.get(slot)
        if hit is not None and hit[0] == key and hit[1].device == device:
            if torch.cuda.is_current_stream_capturing():
                # a graph now reads this table's memory: keep it for the life of the optimizer,
                # even after a later eager step with moved tensors replaces the slot's table
                kept = getattr(self, "_captured_tables", None)
                if kept is None:
                    kept = self._captured_tables = {}
                kept[id(hit[1])] = hit[1]
            return hit[1]
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                "Muon.step under graph capture: a weight, gradient or state tensor moved since "
                "the last eager step (its pointer table would be copied from a temporary host "
                "buffer); run one eager step with the same tensors before capturing")
        table = _pinned_ptrs(list(key), device)
        self._ptr_tables[slot] = (key, table)
        return table

    def _run_pipeline(self, chunks, dev, main, args) -> None:
        """The chunks one after another on ``main``; with ``overlap_staging`` chunk k+1 is
        staged on a side stream into the other workspace while chunk k's NS runs."""
        overlap = self._overlap_staging and len(chunks) > 1
        side = self._side_stream(dev) if overlap else main
        # both workspaces exist before the hand-over event, so no block the side stream writes
        # can still be in use by later work on `main`
        nslots = 2 if overlap else 1
        wss = [self._get_workspace(dev, max(c[8] for k, c in enumerate(chunks)
                                            if k % nslots == sl), sl)
               for sl in range(min(nslots, len(chunks)))]
        if overlap:
            start = torch.cuda.Event()
            start.record(main)           # gradients, buffers and weights are ready on `main`
            side.wait_event(start)
        free = [None, None]
        for k, chunk in enumerate(chunks):
            slot = k % nslots
            ws = wss[slot]
            if free[slot] is not None:
                side.wait_event(free[slot])
            self._stage_chunk(chunk, ws, side, args)
            if overlap:
                staged = torch.cuda.Event()
                staged.record(side)
                main.wait_event(staged)
            self._apply_chunk(chunk, ws, main, args)
            if overlap:
                done = torch.cuda.Event()
                done.record(main)
                free[slot] = done

    def _chunk_sizes(self, rows: int, cols: int, L: int, num_cus: int, backend: int) -> list:
        """Split a bucket of L same-shape matrices into chunks whose NS workspace fits
        ``workspace_limit_bytes``: the fewest chunks, or a few more when that wastes less of the
        last wave of tiles. Cost of a split = sum over chunks of the waves its triangle products
        take (tiles / tiles resident at once, rounded up; a 128-tile wave counts 0.675 of a
        256-tile wave, the library's own tile-choice model), the launches that dominate both NS
        forms."""
        per = _C.plan(rows, cols, 1, 0, num_cus, backend)[3]
        most = max(1, min(L, self._workspace_limit // max(per, 1)))
        while most > 1 and _C.plan(rows, cols, most, 0, num_cus, backend)[3] > \
                self._workspace_limit:
            most -= 1

        def waves(size: int) -> float:
            tile, m_pad, _, _ = _C.plan(rows, cols, size, 0, num_cus, backend)
            mt = m_pad // tile
            tiles = size * mt * (mt + 1) // 2
            if tile == 256:
                return float(-(-tiles // num_cus))
            return 0.675 * (-(-tiles // (2 * num_cus)))

        best = None
        n_min = -(-L // most)
        for n in range(n_min, min(L, n_min + 3) + 1):
            sizes = [L // n + (1 if i < L % n else 0) for i in range(n)]
            cost = sum(waves(sz) for sz in sizes)
            if best is None or cost < best[0] - 1e-9:
                best = (cost, sizes)
        return best[1]

    def _get_workspace(self, device, nbytes: int, slot: int = 0) -> Tensor:
        ws = self._workspaces[slot]
        if ws is None or ws.device != device or ws.numel() < nbytes:
            self._workspaces[slot] = None
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            self._workspaces[slot] = ws
        return ws

    def _side_stream(self, device) -> "torch.cuda.Stream":
        s = self._side_streams.get(device)
        if s is None:
            s = torch.cuda.Stream(device=device)       # default priority
            self._side_streams[device] = s
        return s

    # ------------------------------------------------------------------ AdamW
    def _step_adamw_group(self, group) -> None:
        """Decoupled AdamW, bucketed by (step, param dtype, device, grad dtype) as in
        ``muon.py:1857-1916``; each bucket is one fused HIP pass (``fused_adamw_``)."""
        lr = group["lr"]
        beta1, beta2 = group["betas"]
        wd = group["weight_decay"]
        eps = group["eps"]
        buckets: dict = {}
        for p in group["params"]:
            dp = self._dp_by_param.get(id(p))
            grad = dp.current_grad() if dp is not None else p.grad
            if grad is None:
                continue
            key_obj = id(dp) if dp is not None else p
            # a dedicated param updates its master (_owned_data) and publishes the forward copy
            param = dp._owned_data if dp is not None else p.data
            pub = dp.publish_target() if dp is not None else None
            state = self.state[key_obj]
            if len(state) == 0:
                state["step"] = 0
                state["exp_avg"] = torch.zeros_like(param)
                state["exp_avg_sq"] = torch.zeros_like(param)
            else:
                name = dp.param_name if dp is not None else f"param{tuple(param.shape)}"
                for k in ("exp_avg", "exp_avg_sq"):
                    state[k] = _state_tensor(state[k], tuple(param.shape), param.device,
                                             param.dtype, k, name)
                state["step"] = int(state["step"])
            state["step"] += 1
            key = (state["step"], param.dtype, param.device, grad.dtype,
                   None if pub is None else pub.dtype)
            buckets.setdefault(key, []).append(
                (param, grad, state["exp_avg"], state["exp_avg_sq"], pub))
            if dp is not None:
                dp._reduced_grad = None
        for (step, _pdt, pdev, _gdt, pubdt), items in buckets.items():
            _require_cuda(pdev)
            fused_adamw_([it[0] for it in items], [it[1] for it in items],
                         [it[2] for it in items], [it[3] for it in items], step=step, lr=lr,
                         betas=(beta1, beta2), weight_decay=wd, eps=eps,
                         publish=None if pubdt is None else [it[4] for it in items])

    def zero_grad(self, set_to_none: bool = True):
        self._grads_ready = False
        self._last_muon_grad_clip_stats = None
        for p in self.model.parameters():
            if p.grad is None:
                continue
            if set_to_none:
                p.grad = None
            else:
                p.grad.zero_()
        for dp in self._all_dedicated_params:
            dp._reduced_grad = None
            dp._accumulated_grad = None


def _require_cuda(dev: torch.device) -> None:
    if dev.type != "cuda":
        raise RuntimeError("dmuon_amd.Muon: dedicated parameters must live on the GPU "
                           "(the Muon update runs only on the HIP kernels)")
