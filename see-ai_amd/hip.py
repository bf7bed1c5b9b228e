"""ctypes binding of libseeai_hip.so (include/seeai_hip.h) and the Python
mirror of the reference's executor seam.

``HipBackend`` mirrors ``seeml::update_rt::ExecutorBackend``
(runtime/executor/backend.h:82-166) for the gfx950 executor: ``name``,
``device``, ``Bind``, ``BindSource``, ``Configure``, ``Execute``,
``BeginRange`` / ``EndRange``, ``Flush``, ``relaxed_executions`` -- plus the
host-sync verbs a discrete GPU needs (``Upload`` / ``Download``).  Failures
raise ``BackendError`` carrying the library's message, which for a refused
optimizer step is the reference's own verdict string (backend.h:65-80).

The library is required: importing this module on a machine where it has
not been built raises ``ImportError`` -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import importlib
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libseeai_hip.so")

# torch wheels ship their own libamdhip64.so.7 under the same SONAME as
# ROCm's; whichever loads first serves the whole process.  Load torch's
# first (when torch is installed) so the library and torch share one HIP
# runtime -- loading ours first leaves torch without a usable device.
try:  # noqa: SIM105
    import torch  # noqa: F401
except ImportError:
    pass

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built: run __graft_entry__.build() (hipcc, gfx950)")

_lib = C.CDLL(LIB_PATH)

_P = C.c_void_p
_U64 = C.c_uint64
_I = C.c_int
_F = C.c_float

OK, REFUSED, INVALID, HIP_ERROR = 0, 1, 2, 3

# The reference's shared refusal strings (runtime/executor/backend.h:65-80).
NON_FINITE_NORM_REFUSAL = (
    "gradient norm is not finite — the step was refused with the parameters "
    "and optimizer state untouched")
CLIP_THRESHOLD_REFUSAL = (
    "clip threshold is not a finite positive float — the instruction was "
    "refused with the gradient untouched")


class StepParams(C.Structure):
    """StepParams (runtime/executor/backend.h:56-63)."""
    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("eps", C.c_float), ("weight_decay", C.c_float),
                ("reserved", C.c_uint32), ("step", C.c_uint64)]


class TilePolicy(C.Structure):
    """seeai_tile_policy: the gfx950 kernel geometry (fields as in
    see-ai_amd/policy.py; 0 keeps a default)."""
    _fields_ = [("w8a8_large_kernel", C.c_uint32), ("w8a8_large_min", C.c_uint32),
                ("quantize_waves_per_cu", C.c_uint32), ("relaxed_min_tiles_256", C.c_uint32),
                ("relaxed_min_fill_256", C.c_uint32), ("relaxed_nt_dma_min_k", C.c_uint32),
                ("convert_wgs_per_cu", C.c_uint32),
                ("exact_longk_first", C.c_uint32), ("relaxed_tile_192", C.c_uint32)]


# Every exported symbol with its ctypes signature: the header, one to one.
EXPORTS = {
    "seeai_create": (_I, [_I, C.POINTER(_P)]),
    "seeai_destroy": (None, [_P]),
    "seeai_last_error": (C.c_char_p, [_P]),
    "seeai_set_stream": (_I, [_P, _P]),
    "seeai_get_stream": (_P, [_P]),
    "seeai_set_relaxed": (_I, [_P, _I]),
    "seeai_set_attention_bf16": (_I, [_P, _I]),
    "seeai_relaxed_executions": (_U64, [_P]),
    "seeai_bind": (_I, [_P, _U64, _P, _U64]),
    "seeai_bind_source": (_I, [_P, _P, _U64]),
    "seeai_upload": (_I, [_P, _U64, _P, _U64]),
    "seeai_feeder_create": (_I, [_P, _U64, _U64, _P]),
    "seeai_feeder_destroy": (None, [_P]),
    "seeai_feeder_last_error": (C.c_char_p, [_P]),
    "seeai_feeder_stage": (_I, [_P, _P, _P]),
    "seeai_feeder_next": (_I, [_P, _U64, _U64]),
    "seeai_download": (_I, [_P, _U64, _P, _U64]),
    "seeai_arena": (_P, [_P]),
    "seeai_arena_bytes": (_U64, [_P]),
    "seeai_execute": (_I, [_P, _P, _P]),
    "seeai_execute_range": (_I, [_P, _P, _U64, _P, C.POINTER(_U64)]),
    "seeai_begin_range": (_I, [_P, _P, _U64, _U64, _U64]),
    "seeai_end_range": (_I, [_P]),
    "seeai_run_range": (_I, [_P, _P, _U64, _U64, _U64, _P, C.POINTER(_U64)]),
    "seeai_set_graph_replay": (_I, [_P, _I]),
    "seeai_graph_launches": (_U64, [_P]),
    "seeai_set_fusion": (_I, [_P, _I]),
    "seeai_fused_dispatches": (_U64, [_P]),
    "seeai_dropped_stores": (_U64, [_P]),
    "seeai_fused_conversions": (_U64, [_P]),
    "seeai_flush": (_I, [_P]),
    "seeai_flush_download": (_I, [_P, _U64, _P, _U64]),
    "seeai_configure": (_I, [_P, C.POINTER(TilePolicy)]),
    "seeai_policy": (_I, [_P, C.POINTER(TilePolicy)]),
    "seeai_device_key": (_I, [_I, C.c_char_p, _U64]),
    "seeai_gemm_f32": (_I, [_P, _I, _P, _P, _P, _U64, _U64, _U64, _P, _I, _P, _F, _I]),
    "seeai_gemm_q8": (_I, [_P, _I, _P, _P, _P, _U64, _U64, _U64, _F, _P, _I]),
    "seeai_gemm_bf16w": (_I, [_P, _I, _P, _P, _P, _U64, _U64, _U64, _P, _I]),
    "seeai_w8a8_quantize_rows": (_I, [_P, _P, _P, _P, _U64, _U64]),
    "seeai_w8a8_pack_weights": (_I, [_P, _P, _P, _P, _U64, _U64]),
    "seeai_w8a8_gemm": (_I, [_P, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64]),
    "seeai_attn_fwd": (_I, [_P, _I, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64, _P]),
    "seeai_attn_fwd_bf16": (_I, [_P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64, _P]),
    "seeai_attn_dq_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64]),
    "seeai_attn_dkdv_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64]),
    "seeai_attn_dq": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64]),
    "seeai_attn_dk": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64]),
    "seeai_attn_dv": (_I, [_P, _I, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64]),
    "seeai_attn_dkdv": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64]),
    "seeai_attn_dkdv_f32": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64]),
    "seeai_xent_fwd": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _I]),
    "seeai_xent_fwd_noalloc": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _I]),
    "seeai_xent_bwd": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _I]),
    "seeai_adamw_step": (_I, [_P, _P, _P, _P, _P, _U64, C.POINTER(StepParams), _F]),
    "seeai_argmax_rows": (_I, [_P, _P, _U64, _U64, _P]),
    "seeai_argmax_tally": (_I, [_P, _P, _P, _U64, _U64, C.POINTER(_U64), C.POINTER(_U64)]),
}
# include/seeai_engine.h: the plan engine (see-ai_amd/host/).
ENGINE_EXPORTS = {
    "seeai_plan_self_hash": (_U64, [_P, _U64, _U64]),
    "seeai_plan_check": (_I, [_P, _U64, _P, _U64]),
    "seeai_engine_create": (_I, [_I, _P, _U64, C.POINTER(_P), _P, _U64]),
    "seeai_engine_destroy": (None, [_P]),
    "seeai_engine_last_error": (C.c_char_p, [_P]),
    "seeai_engine_header": (_I, [_P, _P]),
    "seeai_engine_train_step": (_I, [_P, _P, _P, C.POINTER(_F)]),
    "seeai_engine_train_resident": (_I, [_P, C.POINTER(_F)]),
    "seeai_engine_train_steps": (_I, [_P, _P, _P, _U64, _P]),
    "seeai_engine_evaluate": (_I, [_P, _P, _P, C.POINTER(_F)]),
    "seeai_engine_evaluate_metrics": (_I, [_P, _P, _P, C.POINTER(_F), C.POINTER(_U64),
                                          C.POINTER(_U64)]),
    "seeai_engine_merge": (_I, [_P]),
    "seeai_engine_bind_source": (_I, [_P, _P, _U64]),
    "seeai_engine_read": (_I, [_P, _U64, _P, _U64]),
    "seeai_engine_write": (_I, [_P, _U64, _P, _U64]),
    "seeai_engine_step": (_U64, [_P]),
    "seeai_engine_set_step": (None, [_P, _U64]),
    "seeai_engine_set_horizon": (None, [_P, _U64]),
    "seeai_engine_lr": (_F, [_P]),
    "seeai_engine_relaxed_executions": (_U64, [_P]),
    "seeai_engine_context": (_P, [_P]),
}
EXPORTS.update(ENGINE_EXPORTS)
for _name, (_res, _args) in EXPORTS.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


class BackendError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def lib():
    return _lib


def ptr(t) -> int | None:
    """Device address of a torch tensor (or None)."""
    if t is None:
        return None
    return t.data_ptr()


def device_key(device: int = 0) -> str:
    """The device's kernel-policy table key (the GPU's HostKey)."""
    buf = C.create_string_buffer(512)
    rc = _lib.seeai_device_key(device, buf, _U64(512))
    if rc != OK:
        raise BackendError(rc, f"seeai_device_key({device}) failed with status {rc}")
    return buf.value.decode("utf-8", "replace")


def _policy_struct(policy) -> "TilePolicy | None":
    if policy is None:
        return None
    if isinstance(policy, TilePolicy):
        return policy
    return TilePolicy(**{k: int(v) for k, v in policy.items()})


def _configure(ctx_handle, policy):
    p = _policy_struct(policy)
    rc = _lib.seeai_configure(ctx_handle, C.byref(p) if p is not None else None)
    if rc != OK:
        raise BackendError(rc, _lib.seeai_last_error(ctx_handle).decode("utf-8", "replace"))


def _policy_of(ctx_handle) -> dict:
    p = TilePolicy()
    rc = _lib.seeai_policy(ctx_handle, C.byref(p))
    if rc != OK:
        raise BackendError(rc, "seeai_policy failed")
    return {name: int(getattr(p, name)) for name, _ in TilePolicy._fields_}


class Context:
    """One seeai_ctx: a device, a stream, scratch and (optionally) an arena."""

    def __init__(self, device: int = 0):
        h = _P()
        rc = _lib.seeai_create(device, C.byref(h))
        if rc != OK:
            raise BackendError(rc, f"seeai_create failed with status {rc}")
        self.h = h
        self.device_index = device

    def close(self):
        if self.h:
            _lib.seeai_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass

    def check(self, rc: int):
        if rc != OK:
            raise BackendError(rc, _lib.seeai_last_error(self.h).decode("utf-8", "replace"))

    def call(self, name: str, *args):
        self.check(getattr(_lib, name)(self.h, *args))

    def configure(self, policy=None):
        """seeai_configure: a policy dict (see-ai_amd/policy.py fields), a
        TilePolicy, or None for the defaults."""
        _configure(self.h, policy)

    def policy(self) -> dict:
        return _policy_of(self.h)

    def use_torch_stream(self):
        """Enqueue on torch's current stream (0 is the null stream) so torch's
        copies and the library's kernels are ordered."""
        import torch
        handle = torch.cuda.current_stream().cuda_stream
        self.check(_lib.seeai_set_stream(self.h, _P(handle) if handle else None))


class HipBackend:
    """The gfx950 ExecutorBackend (runtime/executor/backend.h:82-166)."""

    def __init__(self, device: int = 0):
        self.ctx = Context(device)
        self._params = StepParams(0.0, 0.9, 0.999, 1e-8, 0.0, 0, 0)

    # backend.h:84-85
    def name(self) -> str:
        return "hip"

    def device(self) -> str:
        return f"AMD gfx950 device {self.ctx.device_index}"

    # backend.h:99-109
    def Bind(self, arena: bytes | bytearray | None, arena_bytes: int, rodata: bytes,
             rodata_bytes: int | None = None):
        ro = bytes(rodata) if rodata is not None else b""
        n = len(ro) if rodata_bytes is None else rodata_bytes
        buf = C.create_string_buffer(ro, max(n, 1))
        self.ctx.call("seeai_bind", _U64(arena_bytes), buf, _U64(n))
        if arena is not None and len(arena):
            self.Upload(0, bytes(arena))

    def BindSource(self, data: bytes | None):
        if not data:
            self.ctx.call("seeai_bind_source", None, _U64(0))
            return
        buf = C.create_string_buffer(bytes(data), len(data))
        self.ctx.call("seeai_bind_source", buf, _U64(len(data)))

    def Configure(self, policy=None):
        """backend.h:117, called after every successful Bind: the gfx950
        member of the kernel-policy table (a dict from policy.resolve), or
        None for the built-in geometry.  The plan header's CPU tiles
        (gemm_tile_k / n) do not apply to this backend."""
        self.ctx.configure(policy)

    def Execute(self, instruction: bytes, params: StepParams | None = None):
        assert len(instruction) == 64
        buf = C.create_string_buffer(bytes(instruction), 64)
        self.ctx.call("seeai_execute", buf, C.byref(params or self._params))

    def ExecuteRange(self, program: bytes, params: StepParams | None = None):
        n = len(program) // 64
        buf = C.create_string_buffer(bytes(program), max(len(program), 1))
        failed = _U64(0)
        rc = _lib.seeai_execute_range(self.ctx.h, buf, _U64(n), C.byref(params or self._params),
                                      C.byref(failed))
        if rc != OK:
            raise BackendError(rc, f"backend 'hip' failed at instruction {failed.value}: "
                               + _lib.seeai_last_error(self.ctx.h).decode("utf-8", "replace"))

    def BeginRange(self, program, begin, end):  # backend.h:139
        return None

    def EndRange(self):
        return None

    def Flush(self):
        self.ctx.call("seeai_flush")

    def relaxed_executions(self) -> int:
        return int(_lib.seeai_relaxed_executions(self.ctx.h))

    def fused_dispatches(self) -> int:  # backend.h:165
        return int(_lib.seeai_fused_dispatches(self.ctx.h))

    def dropped_stores(self) -> int:
        return int(_lib.seeai_dropped_stores(self.ctx.h))

    def fused_conversions(self) -> int:
        return int(_lib.seeai_fused_conversions(self.ctx.h))

    def SetFusion(self, allow: bool):
        self.ctx.call("seeai_set_fusion", int(bool(allow)))

    def SetRelaxed(self, allow: bool):
        self.ctx.call("seeai_set_relaxed", int(bool(allow)))

    def SetAttentionBf16(self, on: bool):
        """Relaxed attention on bf16 operands (True) or f32 products (False,
        the default)."""
        self.ctx.call("seeai_set_attention_bf16", int(bool(on)))

    # host-sync verbs
    def Upload(self, offset: int, data: bytes):
        buf = C.create_string_buffer(bytes(data), max(len(data), 1))
        self.ctx.call("seeai_upload", _U64(offset), buf, _U64(len(data)))

    def Download(self, offset: int, nbytes: int) -> bytes:
        buf = C.create_string_buffer(max(nbytes, 1))
        self.ctx.call("seeai_download", _U64(offset), buf, _U64(nbytes))
        return buf.raw[:nbytes]

    def arena_ptr(self) -> int:
        return _lib.seeai_arena(self.ctx.h)


def pack_instruction(opcode: int, flags: int = 0, imm: int = 0, ins=(), outs=()) -> bytes:
    """One 64-byte UpdateInstruction (source/plan/instruction.h:438-447)."""
    null = 0xFFFFFFFFFFFFFFFF
    i4 = list(ins) + [null] * (4 - len(ins))
    o3 = list(outs) + [0] * (3 - len(outs))
    return struct.pack("<HHI4Q3Q", opcode, flags, imm, *i4, *o3)


def _view(blob) -> "np.ndarray":
    """A uint8 view of any buffer (bytes, bytearray, memoryview) without a
    copy; its .ctypes.data is the address the C ABI reads."""
    import numpy as np
    v = np.frombuffer(blob, np.uint8) if len(blob) else np.zeros(1, np.uint8)
    return v


def plan_self_hash(blob, hash_offset: int = 216) -> int:
    """PlanSelfHash (source/identity/hash.h:136-158) of a plan blob."""
    v = _view(blob)
    return int(_lib.seeai_plan_self_hash(v.ctypes.data, _U64(len(blob)), _U64(hash_offset)))


def plan_check(blob: bytes) -> str:
    """The loader's header contract on a blob: '' if readable, else the
    reference's refusal message (runtime/loader/plan_loader.cc:19-49)."""
    v = _view(blob)
    msg = C.create_string_buffer(512)
    _lib.seeai_plan_check(v.ctypes.data, _U64(len(blob)), msg, _U64(512))
    return msg.value.decode("utf-8", "replace")


class Engine:
    """A loaded plan on one device (include/seeai_engine.h): the reference's
    UpdateEngine verbs over the gfx950 HipBackend."""

    def __init__(self, blob: bytes, device: int = 0):
        v = _view(blob)
        h = _P()
        msg = C.create_string_buffer(512)
        rc = _lib.seeai_engine_create(device, v.ctypes.data, _U64(len(blob)), C.byref(h), msg,
                                      _U64(512))
        if rc != OK:
            raise BackendError(rc, msg.value.decode("utf-8", "replace"))
        self.h = h

    def close(self):
        if self.h:
            _lib.seeai_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass

    def _check(self, rc: int):
        if rc != OK:
            raise BackendError(rc, _lib.seeai_engine_last_error(self.h).decode("utf-8", "replace"))

    def header(self) -> bytes:
        buf = C.create_string_buffer(320)
        self._check(_lib.seeai_engine_header(self.h, buf))
        return buf.raw

    def train_step(self, inputs, labels=None) -> float:
        import numpy as np
        x = np.ascontiguousarray(inputs, np.float32)
        lab = None if labels is None else np.ascontiguousarray(labels)
        loss = _F(0.0)
        self._check(_lib.seeai_engine_train_step(
            self.h, x.ctypes.data, None if lab is None else lab.ctypes.data, C.byref(loss)))
        return loss.value

    def train_steps(self, inputs, labels=None):
        """Optimizer steps over consecutive batches (inputs[b], labels[b]),
        the next batch's upload overlapping the current step; returns one
        loss per step."""
        import numpy as np
        x = np.ascontiguousarray(inputs, np.float32)
        lab = None if labels is None else np.ascontiguousarray(labels)
        batches = x.shape[0]
        pw = importlib.import_module("see-ai_amd.planwriter")
        fields = dict(zip(pw.HEADER_NAMES, struct.unpack(pw.HEADER_FORMAT, self.header())))
        micro = max(1, fields["grad_accum_steps"])
        losses = np.zeros(batches // micro, np.float32)
        self._check(_lib.seeai_engine_train_steps(
            self.h, x.ctypes.data, None if lab is None else lab.ctypes.data, batches,
            losses.ctypes.data))
        return losses

    def train_resident(self) -> float:
        loss = _F(0.0)
        self._check(_lib.seeai_engine_train_resident(self.h, C.byref(loss)))
        return loss.value

    def evaluate(self, inputs, labels=None) -> float:
        import numpy as np
        x = np.ascontiguousarray(inputs, np.float32)
        lab = None if labels is None else np.ascontiguousarray(labels)
        loss = _F(0.0)
        self._check(_lib.seeai_engine_evaluate(
            self.h, x.ctypes.data, None if lab is None else lab.ctypes.data, C.byref(loss)))
        return loss.value

    def evaluate_metrics(self, inputs, labels=None):
        """(loss, hits, judged): the eval program and its accuracy tally."""
        import numpy as np
        x = np.ascontiguousarray(inputs, np.float32)
        lab = None if labels is None else np.ascontiguousarray(labels)
        loss, hits, judged = _F(0.0), _U64(0), _U64(0)
        self._check(_lib.seeai_engine_evaluate_metrics(
            self.h, x.ctypes.data, None if lab is None else lab.ctypes.data, C.byref(loss),
            C.byref(hits), C.byref(judged)))
        return loss.value, int(hits.value), int(judged.value)

    def merge(self):
        self._check(_lib.seeai_engine_merge(self.h))

    def bind_source(self, data: bytes | None):
        """UpdateEngine::BindSourceModel: the source model's image."""
        n = 0 if data is None else len(data)
        buf = None if not n else C.create_string_buffer(bytes(data), n)
        self._check(_lib.seeai_engine_bind_source(self.h, buf, _U64(n)))

    def read(self, offset: int, nbytes: int) -> bytes:
        buf = C.create_string_buffer(max(nbytes, 1))
        self._check(_lib.seeai_engine_read(self.h, _U64(offset), buf, _U64(nbytes)))
        return buf.raw[:nbytes]

    def write(self, offset: int, data: bytes):
        buf = C.create_string_buffer(bytes(data), max(len(data), 1))
        self._check(_lib.seeai_engine_write(self.h, _U64(offset), buf, _U64(len(data))))

    @property
    def step(self) -> int:
        return int(_lib.seeai_engine_step(self.h))

    @step.setter
    def step(self, value: int):
        _lib.seeai_engine_set_step(self.h, _U64(value))

    def set_horizon(self, steps: int):
        _lib.seeai_engine_set_horizon(self.h, _U64(steps))

    def lr(self) -> float:
        return float(_lib.seeai_engine_lr(self.h))

    def relaxed_executions(self) -> int:
        return int(_lib.seeai_engine_relaxed_executions(self.h))

    def set_relaxed(self, allow: bool):
        """Whether kFlagRelaxed instructions may run relaxed; with False the
        whole plan runs the exact family (source/plan/instruction.h:356-384)."""
        ctx = _lib.seeai_engine_context(self.h)
        rc = _lib.seeai_set_relaxed(ctx, int(bool(allow)))
        if rc != OK:
            raise BackendError(rc, _lib.seeai_last_error(ctx).decode("utf-8", "replace"))

    def set_attention_bf16(self, on: bool):
        """Relaxed attention on bf16 operands (True) or f32 products (False,
        the default): HipBackend.SetAttentionBf16 underneath."""
        ctx = _lib.seeai_engine_context(self.h)
        rc = _lib.seeai_set_attention_bf16(ctx, int(bool(on)))
        if rc != OK:
            raise BackendError(rc, _lib.seeai_last_error(ctx).decode("utf-8", "replace"))

    def fused_dispatches(self) -> int:
        return int(_lib.seeai_fused_dispatches(_lib.seeai_engine_context(self.h)))

    def dropped_stores(self) -> int:
        return int(_lib.seeai_dropped_stores(_lib.seeai_engine_context(self.h)))

    def fused_conversions(self) -> int:
        return int(_lib.seeai_fused_conversions(_lib.seeai_engine_context(self.h)))

    def configure(self, policy=None):
        """The backend's kernel geometry (HipBackend.Configure)."""
        _configure(_lib.seeai_engine_context(self.h), policy)

    def set_graph_replay(self, on: bool):
        """seeai_set_graph_replay on the engine's context: ranges replayed
        from captured HIP graphs from their second run (True) or run
        instruction by instruction (False, the default)."""
        rc = _lib.seeai_set_graph_replay(_lib.seeai_engine_context(self.h), int(bool(on)))
        if rc != OK:
            raise BackendError(rc, "set_graph_replay")

    @property
    def graph_launches(self) -> int:
        return int(_lib.seeai_graph_launches(_lib.seeai_engine_context(self.h)))

    def policy(self) -> dict:
        return _policy_of(_lib.seeai_engine_context(self.h))

    def set_fusion(self, allow: bool):
        """Whether adjacent relaxed dK / dV instructions run as one dispatch."""
        ctx = _lib.seeai_engine_context(self.h)
        rc = _lib.seeai_set_fusion(ctx, int(bool(allow)))
        if rc != OK:
            raise BackendError(rc, _lib.seeai_last_error(ctx).decode("utf-8", "replace"))

    def use_torch_stream(self):
        """Run the engine's kernels on torch's current stream."""
        import torch
        handle = torch.cuda.current_stream().cuda_stream
        ctx = _lib.seeai_engine_context(self.h)
        rc = _lib.seeai_set_stream(ctx, _P(handle) if handle else None)
        if rc != OK:
            raise BackendError(rc, _lib.seeai_last_error(ctx).decode("utf-8", "replace"))
