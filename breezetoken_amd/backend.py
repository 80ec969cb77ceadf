"""Host side of the MI355X GQA attention path, mirroring the reference operator API.

``HipBackend`` exposes the attention part of the reference ``Backend`` protocol
(breezetoken/backends.py:47-51, 657-706) with the same names, argument meaning
and shapes, so the Qwen3.5 attention layers call it unchanged:

* ``attention(q, k, v, scale)``: q (H, D), k/v (S, Hkv, D) -> (H, D) f32
  (eager decode, layers.py:75-80);
* ``attention_fixed(q, k, v, pos, scale)``: k/v the whole (cap, Hkv, D) cache,
  ``pos`` a device int32 (1,) holding the 0-based index of the token being
  decoded, valid length pos + 1 (graph decode, graph.py:55-61).

and adds the operators the reference runs outside the protocol:

* ``attention_prefill(q, k, v, scale, q_offset=0)``: causal GQA over new
  tokens at positions q_offset.., q (S, H, D), k/v (q_offset + S, Hkv, D) ->
  (S, H, D) (the SDPA call of prefill.py:56-68, and with q_offset > 0 the
  banded chunked prefill of qwen36_moe.py:394-428); ``sdpa_prefill`` takes
  those calls' (1, H, S, D) layout;
* ``attention_ragged(...)``: many sequences in one shared cache;
* ``rms_norm(x, w, eps)`` and ``rope(x, cos, sin, pos, rope_dim)``: the
  reference Backend's q/k norm and partial RoPE operators (backends.py:44-62);
* ``attn_prep(...)``: the whole decode-step preparation of an attention layer
  (q/k RMSNorm + RoPE, bf16 cache writes at the device position) in one launch
  (layers.py:58-73, graph.py:41-53);
* ``gdn_decode(q, k, v, g, beta, state, scale, eps)``: the Gated DeltaNet
  one-token step with the f32 state updated in place (backends.py:79-92);
* ``linear(x, w)``: the decode matvec x (K,) f32 . w (K, N) bf16 -> (N,) f32
  of every projection and the vocabulary head (backends.py:36-37).

Every launch goes through libbreezetoken_amd.so on torch's current stream with
no host synchronisation, so the calls can be captured in a hipGraph
(``torch.cuda.graph``).  There is no torch or CPU fallback: a shape or dtype
the kernels do not serve raises ``RuntimeError`` (for ``attention_fixed`` this
is the same signal the reference uses to fall back to eager decode,
backends.py:698 with graph.py:127-133).
"""

from __future__ import annotations

import ctypes
from collections import OrderedDict

import torch

from . import _lib
from ._lib import BT_DTYPE_BF16, BT_DTYPE_F32, check

SERVED_HEAD_DIMS = (64, 128, 256)
SERVED_PREP_DIMS = (64, 128, 256, 512)
SERVED_PREFILL_HEAD_DIMS = (128, 256)
MAX_GROUP = 8


def rope_tables(cap: int, rope_dim: int, theta: float, device: str | torch.device = "cuda"):
    """cos/sin (cap, rope_dim) f32 tables for ``rope``/``attn_prep``, built as
    LayerMixin._rope_tables does (layers.py:26-32): inverse frequencies
    theta^(-i/half), phases position * inverse frequency, both halves equal."""
    half = rope_dim // 2
    inv = theta ** (-torch.arange(0, half, device=device, dtype=torch.float32) / half)
    phases = torch.outer(torch.arange(cap, device=device, dtype=torch.float32), inv)
    freqs = torch.cat((phases, phases), dim=-1)
    return freqs.cos(), freqs.sin()


def decode_unserved(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, device: torch.device | None = None) -> str | None:
    """Why the decode kernels cannot take ``attention(q, k, v, scale)``, or None
    when they can: q (H, D) f32/bf16, k/v equal (S >= 1, Hkv, D) bf16 with
    unit d-stride and identical strides, D in SERVED_HEAD_DIMS, H / Hkv <= 8,
    one sequence's KV extent below 4 GiB, every tensor on ``device`` (a GPU
    device; None checks only that they share one GPU)."""
    if q.ndim != 2 or k.ndim != 3 or v.ndim != 3:
        return "attention expects q (H, D), k/v (S, Hkv, D)"
    if v.shape != k.shape:
        return "k/v must be (S, Hkv, D) with equal shapes"
    heads, dim = q.shape
    groups = k.shape[1]
    if groups < 1 or k.shape[2] != dim or heads % groups:
        return f"q heads {heads} / kv {tuple(k.shape)} do not form a GQA group"
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        return "the MI355X path serves a bf16 KV cache only"
    if q.dtype not in (torch.float32, torch.bfloat16):
        return "q must be f32 or bf16"
    if dim not in SERVED_HEAD_DIMS or heads // groups > MAX_GROUP:
        return f"shape H={heads} Hkv={groups} D={dim} is not served"
    if k.shape[0] < 1:
        return "attention needs at least one key"
    if k.stride(2) != 1 or k.stride() != v.stride():
        return "k/v need unit d-stride and identical strides"
    if k.shape[0] * k.stride(0) * 2 >= 1 << 32:
        return "one sequence's KV extent must stay below 4 GiB"
    want = device if device is not None else q.device
    if want.type != "cuda" or any(t.device != want for t in (q, k, v)):
        return "q/k/v must live on the backend's GPU"
    return None


def prefill_unserved(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_offset: int = 0,
                     device: torch.device | None = None) -> str | None:
    """Why ``attention_prefill(q, k, v, scale, q_offset=q_offset)`` cannot run
    on the prefill kernels, or None when it can: q (S, H, D) f32/bf16, k/v
    equal (q_offset + S, Hkv, D) bf16, unit d-stride, identical k/v strides,
    D in SERVED_PREFILL_HEAD_DIMS, H / Hkv <= 8, all on one GPU."""
    if q.ndim != 3 or k.ndim != 3 or v.shape != k.shape:
        return "prefill expects q (S, H, D), k/v (q_offset + S, Hkv, D)"
    steps, heads, dim = q.shape
    groups = k.shape[1]
    if q_offset < 0 or groups < 1 or k.shape[0] != q_offset + steps or k.shape[2] != dim or heads % groups:
        return "prefill q/k/v shapes do not match (k/v need q_offset + S rows)"
    if q.dtype not in (torch.float32, torch.bfloat16) or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        return "the MFMA prefill serves f32 or bf16 q and bf16 k/v"
    if dim not in SERVED_PREFILL_HEAD_DIMS or heads // groups > MAX_GROUP:
        return f"prefill shape H={heads} Hkv={groups} D={dim} is not served"
    if any(t.stride(2) != 1 for t in (q, k, v)):
        return "prefill needs unit d-stride"
    if k.stride() != v.stride():
        return "k and v need identical strides"
    if any(st <= 0 or st % 8 for st in (q.stride(0), q.stride(1), k.stride(0))) or k.stride(1) < 0 or k.stride(1) % 8:
        return "prefill needs token/head strides in positive multiples of 8 elements"
    if any(t.data_ptr() % 16 for t in (q, k, v)):
        return "prefill needs 16-byte aligned q/k/v"
    nblk = -(-k.shape[0] // 64)
    if (nblk + 1) * 64 * k.stride(0) * 2 > 0xFFFFFFFF or nblk * 64 * dim * 2 > 0xFFFFFFFF:
        return "one kv head's K rows and V^T image must stay below 4 GiB"
    want = device if device is not None else q.device
    if want.type != "cuda" or any(t.device != want for t in (q, k, v)):
        return "q/k/v must live on the backend's GPU"
    return None


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return BT_DTYPE_F32
    if dt == torch.bfloat16:
        return BT_DTYPE_BF16
    raise RuntimeError(f"dtype {dt} is not served (f32 or bf16)")


class HipBackend:
    """MI355X GQA attention backend (decode, fixed-capacity decode, prefill, ragged)."""

    name = "hip"

    def __init__(self, device: str | torch.device = "cuda") -> None:
        dev = torch.device(device)
        if dev.type != "cuda":
            raise ValueError(f"the HIP backend needs a GPU device, got {device!r}")
        if not torch.cuda.is_available():
            raise RuntimeError("no ROCm GPU is visible")
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = str(dev)
        self._dev = dev
        self._family = "cuda"  # torch on ROCm keeps the "cuda" device type
        self._lib = _lib.lib()
        props = torch.cuda.get_device_properties(dev)
        self.num_cus = int(props.multi_processor_count)
        self.arch = getattr(props, "gcnArchName", "")
        self._ws: dict[tuple | str, torch.Tensor] = {}
        # Buffers a captured graph may still point at after a larger one
        # replaced them: kept until close().
        self._retired: list[torch.Tensor] = []
        self._plans: "OrderedDict[tuple, tuple]" = OrderedDict()
        self._pinned_plans: dict[tuple, tuple] = {}
        self._dev_plans: dict[tuple, tuple] = {}

    # ------------------------------------------------------------------ utils
    def _grow(self, key, nbytes: int) -> torch.Tensor:
        """A workspace of at least ``nbytes`` under ``key``.  It only grows; a
        replaced buffer is retired, not freed, because a captured graph may
        still point at it (everything is released by close())."""
        ws = self._ws.get(key)
        if ws is None or ws.numel() < nbytes:
            if ws is not None:
                self._retired.append(ws)
            ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self._dev)
            self._ws[key] = ws
        return ws

    def _workspace(self, heads: int, dim: int, total_splits: int) -> torch.Tensor:
        """Decode partials for ``total_splits`` splits of (heads, dim): one
        buffer per (heads, dim), sized at first use for at least the largest
        single-sequence split count."""
        want = max(total_splits, self._max_splits())
        nbytes = int(self._lib.bt_decode_workspace_bytes(heads, dim, want))
        return self._grow(("decode", heads, dim), nbytes)

    def _max_splits(self) -> int:
        return int(self._lib.bt_decode_pick_splits(1, 1 << 30, self.num_cus))

    def _prefill_workspace(self, steps: int, q_offset: int, heads: int, kv_heads: int, dim: int) -> torch.Tensor:
        """Room for the K and V^T images and, where the library splits the key
        range (short prompts, long cached prefixes), its partials."""
        nbytes = int(self._lib.bt_prefill_split_workspace_bytes(steps, q_offset, heads, kv_heads, dim))
        return self._grow("prefill", nbytes)

    @property
    def tile_tokens(self) -> int:
        """Tokens per decode tile; tile t belongs to split t % num_split."""
        return int(self._lib.bt_decode_tile_tokens())

    def pick_splits(self, kv_heads: int, ctx_len: int) -> int:
        return int(self._lib.bt_decode_pick_splits(kv_heads, ctx_len, self.num_cus))

    def _check_kv(self, k: torch.Tensor, v: torch.Tensor, heads: int, dim: int) -> int:
        if k.ndim != 3 or v.shape != k.shape:
            raise RuntimeError("k/v must be (S, Hkv, D) with equal shapes")
        groups = k.shape[1]
        if k.shape[2] != dim or heads % groups:
            raise RuntimeError(f"q heads {heads} / kv {tuple(k.shape)} do not form a GQA group")
        if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise RuntimeError("the MI355X path serves a bf16 KV cache only")
        if k.device != self._dev or v.device != self._dev:
            raise RuntimeError("k/v must live on the backend's device")
        if k.stride(2) != 1 or k.stride() != v.stride():
            raise RuntimeError("k/v need unit d-stride and identical strides")
        if dim not in SERVED_HEAD_DIMS or heads // groups > MAX_GROUP:
            raise RuntimeError(f"shape H={heads} Hkv={groups} D={dim} is not served")
        if k.shape[0] * k.stride(0) * 2 >= 1 << 32:
            raise RuntimeError("one sequence's KV extent must stay below 4 GiB")
        return groups

    def serves_decode(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
        """True when ``attention(q, k, v, scale)`` runs on the decode kernels;
        False where it would raise for the shape, dtype, layout or device."""
        return decode_unserved(q, k, v, self._dev) is None

    def serves_prefill(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_offset: int = 0) -> bool:
        """True when ``attention_prefill(q, k, v, scale, q_offset=...)`` runs on
        the prefill kernels."""
        return prefill_unserved(q, k, v, int(q_offset), self._dev) is None

    # ----------------------------------------------------------- decode (eager)
    def attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
        """GQA decode attention; q (H, D), k/v (S, Hkv, D) -> (H, D) f32 (backends.py:47-51)."""
        if q.ndim != 2 or k.ndim != 3 or v.ndim != 3:
            raise ValueError("attention expects q (H, D), k/v (S, Hkv, D)")
        heads, dim = q.shape
        groups = self._check_kv(k, v, heads, dim)
        seq = k.shape[0]
        if seq < 1:
            raise ValueError("attention needs at least one key")
        return self._decode(q, k, v, scale, groups, seqlen=seq, pos=None, ctx=seq)

    # ------------------------------------------------------ decode (graph path)
    def attention_fixed(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor, scale: float
    ) -> torch.Tensor:
        """Fixed-capacity decode for the graph path (backends.py:682-706).

        k/v are the whole ``(cap, Hkv, D)`` cache; keys ``j <= pos[0]`` are valid.
        Split ranges are derived from ``pos`` on the device, so the launch shape
        is fixed for a given cache and the call can be captured once and replayed.
        """
        if q.ndim != 2 or k.ndim != 3 or v.ndim != 3:
            raise RuntimeError("fixed attention expects q (H, D), k/v (cap, Hkv, D)")
        heads, dim = q.shape
        groups = self._check_kv(k, v, heads, dim)
        if pos.dtype != torch.int32:
            pos = pos.reshape(1).to(torch.int32)  # as backends.py:561
        if pos.device != self._dev:
            raise RuntimeError("pos must be a device tensor")
        return self._decode(q, k, v, scale, groups, seqlen=k.shape[0], pos=pos.reshape(-1)[:1],
                            ctx=k.shape[0])

    def _decode(self, q, k, v, scale, groups, *, seqlen: int, pos, ctx: int) -> torch.Tensor:
        heads, dim = q.shape
        if q.dtype not in (torch.float32, torch.bfloat16):
            raise RuntimeError("q must be f32 or bf16")
        if q.device != self._dev:
            raise RuntimeError("q must live on the backend's device")
        q = q.contiguous()
        ns = self.pick_splits(groups, ctx)
        ws = self._workspace(heads, dim, ns)
        out = torch.empty((heads, dim), dtype=torch.float32, device=self._dev)
        rc = self._lib.bt_gqa_decode(
            q.data_ptr(), _dtype_code(q.dtype), heads * dim,
            k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
            None, _ptr(pos), None, seqlen,
            1, heads, groups, dim, ns, float(scale),
            ws.data_ptr(), ws.numel(), out.data_ptr(), BT_DTYPE_F32, heads * dim,
            _stream(self._dev),
        )
        check("bt_gqa_decode", rc)
        return out

    def decode_partials(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, num_split: int,
        pos: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """The split pass alone: (lse (H, NS) log2-domain, part (H, NS, D)) (attention.py:88-166)."""
        heads, dim = q.shape
        groups = self._check_kv(k, v, heads, dim)
        q = q.contiguous()
        lse = torch.empty((heads, num_split), dtype=torch.float32, device=self._dev)
        part = torch.zeros((heads, num_split, dim), dtype=torch.float32, device=self._dev)
        rc = self._lib.bt_gqa_decode_split(
            q.data_ptr(), _dtype_code(q.dtype), heads * dim,
            k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
            None, _ptr(pos), None, k.shape[0],
            1, heads, groups, dim, num_split, float(scale),
            lse.data_ptr(), part.data_ptr(), _stream(self._dev),
        )
        check("bt_gqa_decode_split", rc)
        return lse, part

    def combine(self, lse: torch.Tensor, part: torch.Tensor) -> torch.Tensor:
        """The LSE combine alone (attention.py:168-189): (H, NS), (H, NS, D) -> (H, D) f32."""
        heads, ns, dim = part.shape
        out = torch.empty((heads, dim), dtype=torch.float32, device=self._dev)
        rc = self._lib.bt_gqa_decode_combine(
            lse.contiguous().data_ptr(), part.contiguous().data_ptr(), 1, heads, dim, ns,
            None, None, ns, out.data_ptr(), BT_DTYPE_F32, heads * dim, _stream(self._dev),
        )
        check("bt_gqa_decode_combine", rc)
        return out

    # ---------------------------------------------------------- batched decode
    def attention_batched(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
        seq_offset: torch.Tensor, scale: float, max_len: int,
    ) -> torch.Tensor:
        """B sequences sharing one cache, uniform split count; q (B, H, D), pos (B,) int32,
        seq_offset (B,) int64 first slot of each sequence -> (B, H, D) f32."""
        batch, heads, dim = q.shape
        groups = self._check_kv(k, v, heads, dim)
        q = q.contiguous()
        ns = max(1, self.pick_splits(groups * batch, max_len))
        ws = self._workspace(heads, dim, batch * ns)
        out = torch.empty((batch, heads, dim), dtype=torch.float32, device=self._dev)
        rc = self._lib.bt_gqa_decode(
            q.data_ptr(), _dtype_code(q.dtype), heads * dim,
            k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
            seq_offset.data_ptr(), pos.data_ptr(), None, k.shape[0],
            batch, heads, groups, dim, ns, float(scale),
            ws.data_ptr(), ws.numel(), out.data_ptr(), BT_DTYPE_F32, heads * dim,
            _stream(self._dev),
        )
        check("bt_gqa_decode", rc)
        return out

    # ----------------------------------------------------------- ragged decode
    MAX_HOST_PLANS = 64

    def ragged_plan(self, lens: list[int], kv_heads: int, target_groups: int | None = None):
        """Split plan for a ragged batch from host lengths, as device tables:
        sequence b gets ceil(len_b / T) splits for the smallest token cap T
        whose total fits ``target_groups`` work-groups per kv head (default:
        one round, CUs / kv heads).  Plans are cached per (lens, target), at
        most MAX_HOST_PLANS of them (least recently used first out); a plan
        used while a graph is being captured is kept until close()."""
        if target_groups is None:
            target_groups = max(1, self.num_cus // max(1, kv_heads))
        key = (tuple(int(x) for x in lens), int(target_groups))
        plan = self._pinned_plans.get(key)
        if plan is None:
            plan = self._plans.get(key)
            if plan is not None:
                self._plans.move_to_end(key)
        if plan is None:
            plan = self._host_plan(key)
            self._plans[key] = plan
            while len(self._plans) > self.MAX_HOST_PLANS:
                self._plans.popitem(last=False)
        if torch.cuda.is_current_stream_capturing() and key not in self._pinned_plans:
            self._pinned_plans[key] = plan
            self._plans.pop(key, None)
        return plan

    def _host_plan(self, key):
        lens, target_groups = key
        batch = len(lens)
        cap = sum(max(1, -(-int(x) // 32)) for x in lens)
        lens_c = (ctypes.c_int32 * batch)(*lens)
        work = (ctypes.c_int32 * (4 * cap))()
        base = (ctypes.c_int32 * batch)()
        count = (ctypes.c_int32 * batch)()
        total = ctypes.c_int32()
        n = self._lib.bt_ragged_plan(
            ctypes.addressof(lens_c), batch, int(target_groups), ctypes.addressof(work), cap,
            ctypes.addressof(base), ctypes.addressof(count), ctypes.addressof(total),
        )
        if n < 0:
            check("bt_ragged_plan", n)
        dev = self._dev
        work_t = torch.tensor(list(work)[: 4 * n], dtype=torch.int32).to(dev)
        base_t = torch.tensor(list(base), dtype=torch.int32).to(dev)
        count_t = torch.tensor(list(count), dtype=torch.int32).to(dev)
        return (work_t, n, base_t, count_t, int(total.value))

    def ragged_plan_device(self, seq_len: torch.Tensor, target_groups: int | None = None):
        """The same plan built on the device from the device lengths ``seq_len``
        (B,) int32, on the current stream with no host synchronisation
        (capturable).  Tables are allocated once per (B, target) and kept until
        close(); returns (work, num_work, split_base, split_count, total_splits)
        with num_work = total_splits = the table capacity max(B, target)."""
        batch = int(seq_len.numel())
        if target_groups is None:
            raise ValueError("target_groups is required (CUs / kv heads for one round)")
        cap = max(batch, int(target_groups))
        key = (batch, int(target_groups))
        bufs = self._dev_plans.get(key)
        if bufs is None:
            bufs = (torch.empty((cap, 4), dtype=torch.int32, device=self._dev),
                    torch.empty(batch, dtype=torch.int32, device=self._dev),
                    torch.empty(batch, dtype=torch.int32, device=self._dev),
                    torch.empty(1, dtype=torch.int32, device=self._dev))
            self._dev_plans[key] = bufs
        work, base, count, total = bufs
        if seq_len.dtype != torch.int32 or seq_len.device != self._dev or not seq_len.is_contiguous():
            raise RuntimeError("seq_len must be a contiguous int32 device tensor")
        rc = self._lib.bt_ragged_plan_device(
            seq_len.data_ptr(), batch, int(target_groups), work.data_ptr(), cap, base.data_ptr(),
            count.data_ptr(), total.data_ptr(), _stream(self._dev),
        )
        check("bt_ragged_plan_device", rc)
        return work, cap, base, count, cap

    def attention_ragged(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_offset: torch.Tensor,
        seq_len: torch.Tensor, lens: list[int] | None, scale: float, target_groups: int | None = None,
    ) -> torch.Tensor:
        """Ragged decode: sequence b reads slots [seq_offset[b], seq_offset[b] + seq_len[b]).

        q (B, H, D); seq_offset (B,) int64 and seq_len (B,) int32 on the device.
        ``lens``: the same lengths on the host, used to plan split counts there;
        None plans on the device from ``seq_len`` instead (no host round trip,
        so a decode step over growing sequences can be captured in a graph).
        """
        batch, heads, dim = q.shape
        groups = self._check_kv(k, v, heads, dim)
        if seq_offset.dtype != torch.int64 or seq_len.dtype != torch.int32:
            raise RuntimeError("seq_offset must be int64 and seq_len int32")
        q = q.contiguous()
        if target_groups is None:
            target_groups = max(1, self.num_cus // max(1, groups))
        if lens is None:
            work, n, base, count, total = self.ragged_plan_device(seq_len, target_groups)
        else:
            work, n, base, count, total = self.ragged_plan(lens, groups, target_groups)
        ws = self._workspace(heads, dim, total)
        out = torch.empty((batch, heads, dim), dtype=torch.float32, device=self._dev)
        rc = self._lib.bt_gqa_decode_ragged(
            q.data_ptr(), _dtype_code(q.dtype), heads * dim,
            k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
            seq_offset.data_ptr(), seq_len.data_ptr(), batch, heads, groups, dim,
            work.data_ptr(), n, base.data_ptr(), count.data_ptr(), total, float(scale),
            ws.data_ptr(), ws.numel(), out.data_ptr(), BT_DTYPE_F32, heads * dim,
            _stream(self._dev),
        )
        check("bt_gqa_decode_ragged", rc)
        return out

    # ------------------------------------------------------------------ prefill
    def prefill_images(self, capacity: int, kv_heads: int, head_dim: int) -> "PrefillImages":
        """Persistent K / V^T images for chunked prefill over one cache of
        ``capacity`` slots (see ``PrefillImages``)."""
        return PrefillImages(self, capacity, kv_heads, head_dim)

    def attention_prefill(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
        out_dtype: torch.dtype = torch.float32, q_offset: int = 0, split_keys: bool = True,
        images: "PrefillImages | None" = None,
    ) -> torch.Tensor:
        """Causal GQA prefill: q (S, H, D) are the new tokens at positions
        q_offset .. q_offset + S - 1 (f32, as the reference computes it, or bf16),
        k/v (q_offset + S, Hkv, D) the bf16 cache including them (any token/head
        strides) -> (S, H, D); row i attends keys
        0 .. q_offset + i.  q_offset = 0 is the SDPA call of prefill.py:56-68, a
        positive one the banded-mask chunked prefill of qwen36_moe.py:394-428.
        ``split_keys=False`` hands the library only the image workspace, which keeps
        one work-group per query block (for comparisons; results agree to ~1e-6).
        ``images`` (a ``PrefillImages`` of this cache) keeps the K / V^T images
        across the chunks of one sequence, so each call converts only the
        blocks from its own first key on; results equal the call without it."""
        if q.ndim != 3 or k.ndim != 3 or v.shape != k.shape:
            raise ValueError("prefill expects q (S, H, D), k/v (q_offset + S, Hkv, D)")
        steps, heads, dim = q.shape
        groups = k.shape[1]
        q_offset = int(q_offset)
        if q_offset < 0 or k.shape[0] != q_offset + steps or k.shape[2] != dim or heads % groups:
            raise RuntimeError("prefill q/k/v shapes do not match (k/v need q_offset + S rows)")
        if q.dtype not in (torch.float32, torch.bfloat16) or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise RuntimeError("the MFMA prefill serves f32 or bf16 q and bf16 k/v")
        if dim not in SERVED_PREFILL_HEAD_DIMS or heads // groups > MAX_GROUP:
            raise RuntimeError(f"prefill shape H={heads} Hkv={groups} D={dim} is not served")
        for t in (q, k, v):
            if t.stride(2) != 1:
                raise RuntimeError("prefill needs unit d-stride")
        if k.stride() != v.stride():
            raise RuntimeError("k and v need identical strides")
        out = torch.empty((steps, heads, dim), dtype=out_dtype, device=self._dev)
        if images is not None:
            return images._run(q, k, v, scale, out, q_offset, split_keys)
        ws = self._prefill_workspace(steps, q_offset, heads, groups, dim)
        ws_len = ws.numel()
        if not split_keys:
            ws_len = int(self._lib.bt_prefill_workspace_bytes(q_offset + steps, groups, dim))
        rc = self._lib.bt_gqa_prefill(
            q.data_ptr(), _dtype_code(q.dtype), k.data_ptr(), v.data_ptr(), q.stride(0), q.stride(1),
            k.stride(0), k.stride(1), steps, q_offset, heads, groups, dim, float(scale),
            ws.data_ptr(), ws_len, out.data_ptr(), _dtype_code(out_dtype),
            out.stride(0), out.stride(1),
            _stream(self._dev),
        )
        check("bt_gqa_prefill", rc)
        return out

    def sdpa_prefill(
        self, qq: torch.Tensor, kk: torch.Tensor, vv: torch.Tensor, scale: float,
        out_dtype: torch.dtype = torch.float32, q_offset: int = 0, images: "PrefillImages | None" = None,
    ) -> torch.Tensor:
        """Drop-in for the SDPA calls of prefill.py:60-68 (q_offset = 0) and
        qwen36_moe.py:415-423 (q_offset = pos0, head-major cache views):
        qq (1, H, S, D), kk/vv (1, Hkv, q_offset + S, D) -> (1, H, S, D)."""
        out = self.attention_prefill(
            qq[0].transpose(0, 1), kk[0].transpose(0, 1), vv[0].transpose(0, 1), scale, out_dtype,
            q_offset=q_offset, images=images,
        )
        return out.transpose(0, 1).unsqueeze(0)

    # ------------------------------------------ q/k norm, RoPE and cache writes
    def _check_f32_dev(self, name: str, t: torch.Tensor) -> None:
        if t.dtype != torch.float32:
            raise RuntimeError(f"{name} must be f32 (the reference keeps activations in f32)")
        if t.device != self._dev:
            raise RuntimeError(f"{name} must live on the backend's device")

    def _rope_args(self, cos, sin, pos, rope_dim: int):
        if cos is None:
            return None, None, None, 0, 1
        for n, t in (("cos", cos), ("sin", sin)):
            self._check_f32_dev(n, t)
            if t.ndim != 2 or t.shape[1] != rope_dim or not t.is_contiguous():
                raise RuntimeError(f"{n} must be a contiguous (cap, rope_dim) table")
        if sin.shape != cos.shape:
            raise RuntimeError("cos and sin tables differ in shape")
        if pos.dtype != torch.int32:
            pos = pos.reshape(-1).to(torch.int32)
        if pos.device != self._dev:
            raise RuntimeError("pos must be a device tensor")
        return cos, sin, pos.reshape(-1)[:1], int(rope_dim), int(cos.shape[0])

    def _rows(self, x, w, eps, cos, sin, pos, rope_dim) -> torch.Tensor:
        self._check_f32_dev("x", x)
        dim = x.shape[-1]
        if dim not in SERVED_PREP_DIMS:
            raise RuntimeError(f"row length {dim} is not served {SERVED_PREP_DIMS}")
        rows = x.numel() // dim
        xr = x.reshape(rows, dim).contiguous()
        out = torch.empty_like(xr)
        if w is not None:
            self._check_f32_dev("w", w)
            w = w.reshape(-1).contiguous()
        cos, sin, pos, rope_dim, cap = self._rope_args(cos, sin, pos, rope_dim)
        rc = self._lib.bt_rms_norm_rope(
            xr.data_ptr(), dim, rows, dim, _ptr(w), float(eps), _ptr(cos), _ptr(sin), _ptr(pos),
            rope_dim, cap, out.data_ptr(), dim, _stream(self._dev),
        )
        check("bt_rms_norm_rope", rc)
        return out.reshape(x.shape)

    def rms_norm(self, x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
        """RMSNorm over the last dimension with a flat learned weight:
        x * rsqrt(mean(x^2) + eps) * w in f32 (backends.py:44-45, 187-189)."""
        if x.shape[-1] != w.numel():
            raise ValueError(f"rms_norm shape mismatch: x {tuple(x.shape)}, w {tuple(w.shape)}")
        return self._rows(x, w, eps, None, None, None, 0)

    def rope(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor,
             rope_dim: int) -> torch.Tensor:
        """Partial rotate-half RoPE on the leading ``rope_dim`` dimensions at the
        device position ``pos`` (backends.py:54-62, 218-226)."""
        if rope_dim < 2 or rope_dim % 2 or rope_dim > x.shape[-1]:
            raise ValueError(f"invalid rope_dim {rope_dim} for rows of {x.shape[-1]}")
        return self._rows(x, None, 0.0, cos, sin, pos, rope_dim)

    @staticmethod
    def _cache_strides(cache: torch.Tensor, kv_heads: int, dim: int) -> tuple[int, int, int]:
        if cache.dtype != torch.bfloat16 or cache.stride(-1) != 1:
            raise RuntimeError("the cache must be bf16 with unit d-stride")
        if cache.ndim == 2 and cache.shape[1] == kv_heads * dim:
            return cache.shape[0], cache.stride(0), dim
        if cache.ndim == 3 and cache.shape[1:] == (kv_heads, dim):
            return cache.shape[0], cache.stride(0), cache.stride(1)
        raise RuntimeError("the cache must be (cap, Hkv*D) or a (cap, Hkv, D) view")

    def attn_prep(
        self, qkv: torch.Tensor, q_norm: torch.Tensor | None, k_norm: torch.Tensor | None,
        eps: float, cos: torch.Tensor | None, sin: torch.Tensor | None, pos: torch.Tensor,
        rope_dim: int, cache_k: torch.Tensor, cache_v: torch.Tensor, heads: int, kv_heads: int,
        head_dim: int, q_dtype: torch.dtype = torch.float32,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Decode-step preparation of one attention layer (layers.py:58-73,
        graph.py:41-53) in one launch: from the fused projection output ``qkv``
        ([H x (q | gate) | Hkv x k | Hkv x v], f32) write k = rope(rms_norm(k))
        and v into the bf16 caches at slot ``pos`` (device int32) and return
        (q, gate): q = rope(rms_norm(q)) (H, D) in ``q_dtype`` and the gate as
        an (H, D) view of ``qkv``."""
        self._check_f32_dev("qkv", qkv)
        D = int(head_dim)
        if qkv.numel() != heads * 2 * D + 2 * kv_heads * D or heads % kv_heads:
            raise RuntimeError("qkv does not hold H x (q | gate) + 2 x Hkv x D values")
        if D not in SERVED_PREP_DIMS:
            raise RuntimeError(f"head_dim {D} is not served {SERVED_PREP_DIMS}")
        qkv = qkv.reshape(-1).contiguous()
        if (q_norm is None) != (k_norm is None):
            raise RuntimeError("q_norm and k_norm are given together")
        if q_norm is not None:
            self._check_f32_dev("q_norm", q_norm)
            self._check_f32_dev("k_norm", k_norm)
            if q_norm.numel() != D or k_norm.numel() != D:
                raise ValueError("q_norm/k_norm must hold head_dim values")
            q_norm, k_norm = q_norm.reshape(-1).contiguous(), k_norm.reshape(-1).contiguous()
        cos, sin, pos_d, rope_dim, rcap = self._rope_args(cos, sin, pos, rope_dim)
        if pos_d is None:
            pos_d = pos.reshape(-1)[:1]
            if pos_d.dtype != torch.int32 or pos_d.device != self._dev:
                raise RuntimeError("pos must be a device int32 tensor")
        cap, st_tok, st_head = self._cache_strides(cache_k, kv_heads, D)
        if self._cache_strides(cache_v, kv_heads, D) != (cap, st_tok, st_head):
            raise RuntimeError("k and v caches need identical shapes and strides")
        for n, t in (("cache_k", cache_k), ("cache_v", cache_v)):
            if t.device != self._dev:
                raise RuntimeError(f"{n} must live on the backend's device")
        q = torch.empty((heads, D), dtype=q_dtype, device=self._dev)
        rc = self._lib.bt_attn_prep(
            qkv.data_ptr(), heads, kv_heads, D, _ptr(q_norm), _ptr(k_norm), float(eps), _ptr(cos),
            _ptr(sin), pos_d.data_ptr(), rope_dim, rcap, q.data_ptr(), _dtype_code(q_dtype),
            cache_k.data_ptr(), cache_v.data_ptr(), st_tok, st_head, cap, _stream(self._dev),
        )
        check("bt_attn_prep", rc)
        gate = qkv[: heads * 2 * D].view(heads, 2 * D)[:, D:]
        return q, gate

    # ---------------------------------------------------------- decode matvec
    def linear(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """One decode matvec: ``x`` (..., K) f32 times ``w`` (K, N) bf16 -> (N,)
        f32 (backends.py:36-37, 620-630; x.numel() == K as in _torch_linear,
        182-184)."""
        K, N = w.shape
        if x.shape[-1] != K:
            raise ValueError(f"linear shape mismatch: x {tuple(x.shape)}, w {tuple(w.shape)}")
        if x.numel() != K:
            raise ValueError("linear is a matvec: x must hold exactly K values")
        self._check_f32_dev("x", x)
        if w.dtype != torch.bfloat16 or w.device != self._dev or w.stride(1) != 1:
            raise RuntimeError("w must be a bf16 (K, N) device tensor with unit column stride")
        if N % 8 or w.stride(0) % 8 or w.data_ptr() % 16:
            raise RuntimeError("w needs N and its row stride in multiples of 8 and 16-byte alignment")
        x = x.reshape(-1).contiguous()
        nbytes = int(self._lib.bt_gemv_workspace_bytes(K, N))
        ws = None
        if nbytes:
            ws = self._ws.get(("gemv", K, N))
            if ws is None:
                ws = torch.empty(nbytes, dtype=torch.uint8, device=self._dev)
                self._ws[("gemv", K, N)] = ws  # kept: captured graphs may point at it
        y = torch.empty(N, dtype=torch.float32, device=self._dev)
        rc = self._lib.bt_gemv_bf16(x.data_ptr(), w.data_ptr(), w.stride(0), K, N, y.data_ptr(), _ptr(ws),
                                    nbytes, _stream(self._dev))
        check("bt_gemv_bf16", rc)
        return y

    # ------------------------------------------------------------ GDN decode
    def gdn_decode(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
        beta: torch.Tensor, state: torch.Tensor, scale: float, eps: float = 1e-6,
    ) -> torch.Tensor:
        """One gated-delta-rule step; updates ``state`` in place and returns ``o``
        (backends.py:79-92, 242-271).  q/k (Hk, D), v (Hv, D), g/beta (Hv,),
        state (Hv, D, D) f32 contiguous; value head h reads key head h % Hk."""
        if q.shape != k.shape or q.ndim != 2 or v.ndim != 2:
            raise ValueError("q/k must be (key_heads, dim); v must be (value_heads, dim)")
        heads_k, dim = q.shape
        heads_v = v.shape[0]
        if heads_v % heads_k:
            raise ValueError("value_heads must be a multiple of key_heads")
        if state.shape != (heads_v, dim, dim):
            raise ValueError(f"state shape {tuple(state.shape)} != {(heads_v, dim, dim)}")
        for n, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta), ("state", state)):
            self._check_f32_dev(n, t)
        if not state.is_contiguous():
            raise RuntimeError("the GDN state must be contiguous (it is updated in place)")
        if dim not in (64, 128):
            raise RuntimeError(f"GDN decode serves dim 64 or 128, got {dim}")
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        g, beta = g.reshape(-1).contiguous(), beta.reshape(-1).contiguous()
        if g.numel() != heads_v or beta.numel() != heads_v:
            raise ValueError("g and beta need one value per value head")
        out = torch.empty((heads_v, dim), dtype=torch.float32, device=self._dev)
        rc = self._lib.bt_gdn_decode(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), state.data_ptr(),
            heads_k, heads_v, dim, float(scale), float(eps), out.data_ptr(), _stream(self._dev),
        )
        check("bt_gdn_decode", rc)
        return out

    def close(self) -> None:
        self._ws.clear()
        self._retired.clear()
        self._plans.clear()
        self._pinned_plans.clear()
        self._dev_plans.clear()

    def __repr__(self) -> str:
        return f"HipBackend(device={self.device!r}, arch={self.arch!r}, cus={self.num_cus})"


class PrefillImages:
    """The block-scaled fp16 K and V^T images of one layer's cache, kept across
    the chunks of a chunked prefill (qwen36_moe.py:394-428 runs one prefill call
    per chunk at growing ``pos0``): each call converts only the 64-key blocks
    from its own first key on, instead of the whole cached prefix.

    The images are valid for the cache (data pointer and strides) they were
    built from and for keys below ``valid_keys``; a call on another cache, or
    at a ``q_offset`` below ``valid_keys`` (a rewound sequence), rebuilds from
    ``min(valid_keys, q_offset)`` or from 0.  The caller must not change cached
    keys below ``valid_keys`` between calls (``reset()`` forgets them)."""

    def __init__(self, backend: HipBackend, capacity: int, kv_heads: int, head_dim: int) -> None:
        self._be = backend
        self.capacity, self.kv_heads, self.head_dim = int(capacity), int(kv_heads), int(head_dim)
        nbytes = int(backend._lib.bt_prefill_workspace_bytes(self.capacity, self.kv_heads, self.head_dim))
        if nbytes <= 0:
            raise RuntimeError("invalid image shape")
        self.buf = torch.empty(nbytes, dtype=torch.uint8, device=backend._dev)
        self.valid_keys = 0
        self._source: tuple | None = None

    def reset(self) -> None:
        self.valid_keys = 0
        self._source = None

    def _run(self, q, k, v, scale, out, q_offset: int, split_keys: bool) -> torch.Tensor:
        be = self._be
        steps, heads, dim = q.shape
        groups = k.shape[1]
        if (groups, dim) != (self.kv_heads, self.head_dim) or q_offset + steps > self.capacity:
            raise RuntimeError("these images were made for another cache shape or capacity")
        source = (k.data_ptr(), v.data_ptr(), tuple(k.stride()))
        cached = min(self.valid_keys, q_offset) if source == self._source else 0
        pbytes = int(be._lib.bt_prefill_partials_bytes(steps, q_offset, heads, groups, dim)) if split_keys else 0
        part = be._grow("prefill_partials", pbytes) if pbytes else None
        rc = be._lib.bt_gqa_prefill_cached(
            q.data_ptr(), _dtype_code(q.dtype), k.data_ptr(), v.data_ptr(), q.stride(0), q.stride(1),
            k.stride(0), k.stride(1), steps, q_offset, heads, groups, dim, float(scale),
            self.buf.data_ptr(), self.buf.numel(), self.capacity, cached,
            _ptr(part), pbytes, out.data_ptr(), _dtype_code(out.dtype), out.stride(0), out.stride(1),
            _stream(be._dev),
        )
        check("bt_gqa_prefill_cached", rc)
        self._source = source
        self.valid_keys = q_offset + steps
        return out


def make_backend(kind: str = "hip", device: str = "cuda") -> HipBackend:
    """Factory in the spirit of ``make_backend`` (backends.py:860-903) for this path."""
    if kind not in ("hip", "auto"):
        raise ValueError(f"unknown backend {kind!r}")
    return HipBackend(device)
