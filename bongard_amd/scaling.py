"""Delayed (amax-history) scaling for the FP8 path.

Semantics are TransformerEngine's ``DelayedScaling`` with margin 0 and
``amax_compute_algo='max'`` (the reference reaches TE only through Float8CurrentScaling,
bongard/te_linear.py:38-39; delayed scaling is the extension BASELINE config 5 asks for):
a tensor role quantized at step t uses ``scale_t = fp8_max / max(history)``, where the
history holds the amaxes of the previous ``length`` quantizations of that role; while
the history is all zero (or holds a non-finite value) the previous scale is kept, and
the first scale is 1.

On the GPU a delayed quantization is one kernel (``bf8_cast_delayed_bf16``): it folds the
previous step's amax partials into the history, derives the scale, casts, and writes
this step's amax partials, which the next quantization of the role folds in. No amax
pre-pass and no host synchronisation are needed.
"""

import weakref
from collections import deque

import torch

from . import ops
from .ops import E4M3, E5M2

DEFAULT_HISTORY = 16


def _saved_tensor_hook_stack():
    """The saved-tensor default hooks in effect, innermost first, as (pack, unpack) pairs.
    torch exposes only the top of the stack, so the stack is popped and pushed back in
    order (nothing runs in between). Raises if the stack cannot be read: delayed scaling
    must not guess whether it runs in a checkpoint replay."""
    ag = torch._C._autograd
    try:
        if not ag._saved_tensors_hooks_is_enabled():
            return []       # disabled: no region can have pushed hooks either
        popped = []
        try:
            while True:
                top = ag._top_saved_tensors_default_hooks(False)
                if top is None:
                    break
                ag._pop_saved_tensors_default_hooks()
                popped.append(top)
        finally:
            for pack, unpack in reversed(popped):
                ag._push_saved_tensors_default_hooks(pack, unpack)
        return popped
    except (AttributeError, TypeError) as e:
        raise RuntimeError("delayed scaling: this torch build does not expose the "
                           "saved-tensor hook stack, so a checkpoint replay cannot be "
                           "recognised") from e


def _closure(fn):
    code = getattr(fn, "__code__", None)
    if code is None or not fn.__closure__:
        return {}
    return dict(zip(code.co_freevars, (c.cell_contents for c in fn.__closure__)))


def checkpoint_region(forward_role=True):
    """``(frame, recomputing)`` of the non-reentrant ``torch.utils.checkpoint`` region the
    current call runs in: ``frame`` identifies the region (None outside one) and
    ``recomputing`` is True while backward replays the region's forward. The reference
    trains with non-reentrant checkpointing of every text layer (bongard/model.py:124-132,
    234-247), so a delayed-scaling forward runs twice per step: the replay must quantize
    with the scales of the original call and leave the histories alone.

    The region is read from the saved-tensor hooks torch.utils.checkpoint installs (its
    pack hook closes over the region's frame): the innermost of them on the hook stack, so
    other hooks pushed inside the region (CPU offload of activations, say) do not hide it.
    A forward that runs inside a backward pass with no such hook around it is a replay this
    cannot attribute (reentrant checkpointing re-runs forwards that way): for a forward
    tensor role (``forward_role``; gradient roles are quantized inside backward by design)
    that raises."""
    for pack, _ in _saved_tensor_hook_stack():
        name = getattr(pack, "__qualname__", "")
        if name.startswith("_recomputation_hook"):
            ref = _closure(pack).get("target_frame_ref")
            return (ref() if ref is not None else None), True
        if name.startswith("_checkpoint_hook"):
            return _closure(pack).get("frame"), False
    if forward_role and torch._C._current_graph_task_id() != -1:
        raise RuntimeError(
            "delayed scaling: an FP8 forward runs inside a backward pass outside a "
            "non-reentrant torch.utils.checkpoint region (a reentrant checkpoint replay?); "
            "its scales would advance as for a new step. Use "
            "torch.utils.checkpoint.checkpoint(..., use_reentrant=False).")
    return None, False


class DelayedScaler:
    """Delayed scaling state of one tensor role (e.g. a linear's input)."""

    def __init__(self, fmt, history=DEFAULT_HISTORY, *, gradient=False):
        if fmt not in (E4M3, E5M2):
            raise ValueError(f"bad fp8 format {fmt}")
        if not 1 <= int(history) <= 1024:
            raise ValueError("amax history length must be in [1, 1024]")
        self.fmt = fmt
        self.gradient = bool(gradient)   # quantized in backward (grad_output roles)
        self.length = int(history)
        self.state = None     # device float32 [length + 4]: history, meta
        self.recorded = 0     # amaxes pushed into the history so far
        self._bufs = [None, None]
        self._slot = 0        # buffer for this step's partials; the other one is pending
        self._pending = 0     # partial count of the previous step (0: none)
        # checkpointed forwards: per region, the metas of its calls in call order, which the
        # region's replay takes back in the same order (dropped with the region)
        self._records = weakref.WeakKeyDictionary()

    def _ensure(self, device):
        if self.state is None:
            self.state = ops.new_delayed_state(self.length, device)
        elif self.state.device != device:
            self.state = self.state.to(device)
            self._bufs = [None, None]
            self._pending = 0

    def _buffer(self, slot, count, device):
        buf = self._bufs[slot]
        if buf is None or buf.numel() < count or buf.device != device:
            buf = torch.empty(max(int(count), 1024), dtype=torch.int32, device=device)
            self._bufs[slot] = buf
        return buf[:count]

    def partials_for_producer(self, count, device):
        """Buffer the producer of the role's next tensor fills with its amax partials (the
        gated-GELU GEMM for H, its backward for dGU); pass ``count`` to :meth:`quantize`."""
        self._ensure(device)
        return self._buffer(self._slot, count, device)

    def _remember(self, frame, meta):
        if frame is not None:
            self._records.setdefault(frame, deque()).append(meta)

    def _recorded_meta(self, frame):
        calls = self._records.get(frame) if frame is not None else None
        if not calls:
            raise RuntimeError(
                "delayed scaling: a checkpointed forward is replayed but its original call "
                "recorded no scale (the replayed region differs from the original one)")
        return calls.popleft()

    def quantize(self, x, *, rowwise=True, transpose=False, producer_count=None):
        """Quantize ``x`` (bf16, flattened to 2-D) with this role's delayed scale.

        A replay of a checkpointed forward casts with the scale its original call used and
        leaves the history, the pending amax partials and the step count unchanged, so the
        backward sees the original bytes."""
        frame, replay = checkpoint_region(not self.gradient)
        if replay:
            meta = self._recorded_meta(frame)
            return ops.cast(x, meta, self.fmt, rowwise=rowwise, transpose=transpose)
        job, count = self._job(x, rowwise, transpose, producer_count)
        q = ops.cast_delayed(x, job["state"], job["length"], job["pos"], job["prev_partials"],
                             self.fmt, rowwise=rowwise, transpose=transpose,
                             partials_out=job["partials_out"])
        self._commit(job, count, frame, q)
        return q

    def _job(self, x, rowwise, transpose, producer_count):
        """The arguments of this role's next delayed cast of ``x`` (a dict for
        ops.cast_delayed_many) and the number of amax partials it leaves pending."""
        dev = x.device
        self._ensure(dev)
        rows = x.numel() // x.shape[-1] if x.dim() else 1
        cols = x.shape[-1]
        if producer_count is None:
            count = ops.cast_amax_partials_count(rows, cols, transpose)
            out_parts = self._buffer(self._slot, count, dev)
        else:
            count, out_parts = int(producer_count), None
        prev = self._bufs[self._slot ^ 1][:self._pending] if self._pending else None
        job = dict(x=x, state=self.state, length=self.length, pos=self.recorded % self.length,
                   prev_partials=prev, fmt=self.fmt, rowwise=rowwise, transpose=transpose,
                   partials_out=out_parts)
        return job, count

    def _commit(self, job, count, frame, q):
        """The bookkeeping after the cast of ``job``: its previous amax entered the
        history, this cast's partials are pending, the region records the meta."""
        if job["prev_partials"] is not None:
            self.recorded += 1
        self._pending = count
        self._slot ^= 1
        self._remember(frame, q.meta)

    def produce(self, count, device, launch, replay=None):
        """Runs a kernel that produces this role's tensor and casts it with the role's
        delayed scale in the same pass: ``launch(state, length, pos, prev_partials,
        partials_out)`` (the arguments of ``cast_delayed``) returns the FP8 tensor (or a
        tuple whose first item is it) and writes ``count`` amax partials of the new tensor
        into ``partials_out``. A replay of a checkpointed forward calls ``replay(meta,
        partials_out)`` instead, with the meta of the original call and a throwaway partials
        buffer, and leaves the role's state unchanged."""
        frame, again = checkpoint_region(not self.gradient)
        if again:
            if replay is None:
                raise RuntimeError("delayed scaling: this producer cannot be replayed")
            scratch = torch.empty(max(int(count), 1), dtype=torch.int32, device=device)
            return replay(self._recorded_meta(frame), scratch)
        self._ensure(device)
        out_parts = self._buffer(self._slot, count, device)
        prev = self._bufs[self._slot ^ 1][:self._pending] if self._pending else None
        q = launch(self.state, self.length, self.recorded % self.length, prev, out_parts)
        if prev is not None:
            self.recorded += 1
        self._pending = int(count)
        self._slot ^= 1
        self._remember(frame, (q[0] if isinstance(q, tuple) else q).meta)
        return q

    def fold_pending(self):
        """Pushes the amax of the last quantization into the history now instead of at the
        next one (which then has nothing to fold): the scales that follow are the same
        either way, and the state tensor alone then describes the role completely."""
        if not self._pending or self.state is None:
            return
        prev = self._bufs[self._slot ^ 1][:self._pending]
        ops.delayed_scale_fold(self.state, self.length, self.recorded % self.length, prev,
                               self.fmt)
        self.recorded += 1
        self._pending = 0

    # -- persistence (``_extra_state``) -------------------------------------------------
    def to_tensor(self):
        """float32 [3 + length + 4] on the CPU: length, amaxes recorded, format, state (the
        last quantization's amax folded into the history first, so that a run resumed from
        this tensor continues with the scales of the uninterrupted one)."""
        self.fold_pending()
        head = torch.tensor([self.length, self.recorded, self.fmt], dtype=torch.float32)
        if self.state is None:
            body = _fresh_state_cpu(self.length)
        else:
            body = self.state.detach().float().cpu()
        return torch.cat([head, body])

    def load_tensor(self, t):
        t = t.detach().float().cpu()
        length, recorded, fmt = int(t[0]), int(t[1]), int(t[2])
        if length != self.length or fmt != self.fmt or t.numel() != 3 + length + 4:
            raise ValueError("delayed-scaling state does not match this role")
        device = self.state.device if self.state is not None else None
        state = t[3:].clone()
        self.state = state.to(device) if device is not None else state
        self.recorded = recorded
        self._pending = 0


def _fresh_state_cpu(length):
    st = torch.zeros(length + 4, dtype=torch.float32)
    st[length + 1] = 1.0
    st[length + 2] = 1.0
    return st


# The most previous partials a shared launch folds inline (bf8_cast_delayed_many_bf16).
_MANY_MAX_PREV = 2048


def quantize_many(requests):
    """Each ``(scaler, x, rowwise, transpose)`` of ``requests`` quantized with its role's
    delayed scale, in one launch: equal to ``scaler.quantize(x, rowwise=..., transpose=...)``
    for each request in order (bytes, metas, histories, partials), which is what a
    checkpoint replay, or a role whose pending partials exceed what one launch folds, runs
    instead. A forward quantizes its input and weights together this way, as TE casts one
    forward's operands together (bongard/te_linear.py:73-74)."""
    if not requests:
        return []
    regions = [checkpoint_region(not sc.gradient) for sc, _, _, _ in requests]
    if any(replay for _, replay in regions) or any(
            sc._pending > _MANY_MAX_PREV for sc, _, _, _ in requests) or len(requests) > 8:
        return [sc.quantize(x, rowwise=rw, transpose=tr) for sc, x, rw, tr in requests]
    jobs = []
    for sc, x, rw, tr in requests:
        jobs.append(sc._job(x, rw, tr, None))
    qs = ops.cast_delayed_many([job for job, _ in jobs])
    for (sc, _, _, _), (job, count), (frame, _), q in zip(requests, jobs, regions, qs):
        sc._commit(job, count, frame, q)
    return qs


class LinearScaling:
    """Delayed scalers of one FP8 linear, as TE keeps per module: its input and weight
    (e4m3, forward) and the gradient of its output (e5m2, backward)."""

    ROLES = ('input', 'weight', 'grad_output')

    def __init__(self, history=DEFAULT_HISTORY):
        self.history = int(history)
        self.input = DelayedScaler(E4M3, history)
        self.weight = DelayedScaler(E4M3, history)
        self.grad_output = DelayedScaler(E5M2, history, gradient=True)

    def to_tensor(self):
        return torch.cat([getattr(self, r).to_tensor() for r in self.ROLES])

    def load_tensor(self, t):
        n = 3 + self.history + 4
        if t.numel() != len(self.ROLES) * n:
            raise ValueError("delayed-scaling state has the wrong size")
        for i, r in enumerate(self.ROLES):
            getattr(self, r).load_tensor(t[i * n:(i + 1) * n])
