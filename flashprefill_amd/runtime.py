"""Host-side driver of the C ABI: builds the ``fp_problem`` descriptor from
torch tensors, owns the workspace (from torch's caching allocator, so it is
stream ordered), launches on torch's current stream, and exposes the
workspace intermediates (pooled K, per-row index lists and counts) as tensor
views for parity checks.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.FP_DTYPE_BF16, torch.float16: _lib.FP_DTYPE_F16,
           torch.float32: _lib.FP_DTYPE_F32}
BLOCK = 128


class _WorkspaceCache:
    """One reusable workspace per (device, stream) for the operator entry
    points, grown as needed, so that a call allocates nothing once the
    largest shape has been seen. Work on one stream is ordered, so calls on
    that stream can share its buffer; calls on different streams get
    different buffers. During HIP-graph capture a fresh buffer is taken from
    the allocator instead (it then belongs to the graph's memory pool)."""

    def __init__(self):
        self._bufs = {}

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        stream = torch.cuda.current_stream(device)
        if torch.cuda.is_current_stream_capturing():
            return torch.empty(nbytes, dtype=torch.uint8, device=device)
        key = (device.index, stream.cuda_stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            grow = nbytes if buf is None else max(nbytes, buf.numel() + buf.numel() // 2)
            self._bufs[key] = buf = None
            buf = torch.empty(grow, dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf

    def clear(self) -> None:
        self._bufs.clear()


WORKSPACES = _WorkspaceCache()


def release_workspaces() -> None:
    """Drop the cached operator workspaces (their memory returns to torch's
    caching allocator)."""
    WORKSPACES.clear()


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype not in _DTYPES:
        raise NotImplementedError(
            f"FlashPrefill GPU path supports bfloat16, float16 and float32 inputs, got {t.dtype}")
    return _DTYPES[t.dtype]


class FlashPrefillCall:
    """One operator invocation on packed (T, H, d) tensors.

    ``cu_seqlens`` is a device int32 tensor of B+1 offsets, or None for
    ``batch`` sequences of ``uniform_seq_len`` tokens (the batched layout).
    The workspace is ``workspace`` when given, else the stream's cached one
    when ``cached_workspace`` is set, else a new allocation.
    """

    def __init__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                 cu_seqlens: Optional[torch.Tensor], max_seq_len: int, *, alpha: float,
                 attention_sink: int = 2, window_size: int = 4, last_n_block: int = 2,
                 native_normalize: bool = False, min_budget: int = 0,
                 block_size: int = BLOCK, batch: Optional[int] = None,
                 uniform_seq_len: int = 0, workspace: Optional[torch.Tensor] = None,
                 cached_workspace: bool = False):
        for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
            if t.dim() != 3:
                raise ValueError(f"{name} must be (tokens, heads, head_dim), got {tuple(t.shape)}")
            if not t.is_cuda:
                raise ValueError(f"{name} must be a GPU tensor")
            if t.stride(-1) != 1:
                raise ValueError(f"{name} must have a contiguous head dimension")
        if not (q.dtype == k.dtype == v.dtype == o.dtype):
            raise ValueError("q, k, v and o must share one dtype")
        T, Hq, d = q.shape
        Hkv = k.shape[1]
        if k.shape != v.shape or k.shape[0] != T or k.shape[2] != d or o.shape != q.shape:
            raise ValueError(f"shape mismatch: q{tuple(q.shape)} k{tuple(k.shape)} "
                             f"v{tuple(v.shape)} o{tuple(o.shape)}")
        self.device = q.device
        self.tensors = (q, k, v, o)
        if cu_seqlens is not None:
            cu_seqlens = cu_seqlens.to(device=self.device, dtype=torch.int32).contiguous()
            batch = cu_seqlens.numel() - 1
        self.cu_seqlens = cu_seqlens
        self.batch = int(batch)
        self.max_seq_len = int(max_seq_len)
        self.Hq, self.Hkv, self.d = Hq, Hkv, d
        # block_size 256: 256-token selection blocks (pooled K, block scores)
        # over a 128-token plan (work items, index lists, attention)
        self.block = int(block_size)
        self.ratio = 2 if self.block == 256 else 1
        P = _lib.FpProblem()
        P.q, P.k, P.v, P.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
        P.q_stride_tok, P.q_stride_head = q.stride(0), q.stride(1)
        P.k_stride_tok, P.k_stride_head = k.stride(0), k.stride(1)
        P.v_stride_tok, P.v_stride_head = v.stride(0), v.stride(1)
        P.o_stride_tok, P.o_stride_head = o.stride(0), o.stride(1)
        P.cu_seqlens = cu_seqlens.data_ptr() if cu_seqlens is not None else None
        P.batch = self.batch
        P.uniform_seq_len = int(uniform_seq_len)
        P.max_seq_len = self.max_seq_len
        P.total_tokens = T
        P.num_q_heads, P.num_kv_heads, P.head_dim = Hq, Hkv, d
        P.dtype = _dtype_code(q)
        P.block_size = int(block_size)
        P.alpha = float(alpha)
        P.attention_sink = int(attention_sink)
        P.window_size = int(window_size)
        P.last_n_block = int(last_n_block)
        P.native_normalize = 1 if native_normalize else 0
        P.min_budget = int(min_budget)
        self.P = P
        self.lib = _lib.load()
        L = _lib.FpWsLayout()
        _lib.check(self.lib.fp_workspace_layout(ctypes.byref(P), ctypes.byref(L)))
        self.layout = L
        if workspace is None and cached_workspace:
            workspace = WORKSPACES.get(self.device, L.total_bytes)
        if workspace is None or workspace.numel() < L.total_bytes:
            workspace = torch.empty(L.total_bytes, dtype=torch.uint8, device=self.device)
        self.workspace = workspace

    # -- launches ---------------------------------------------------------
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _ws(self) -> int:
        return self.workspace.data_ptr()

    def run(self) -> None:
        _lib.check(self.lib.fp_flashprefill(ctypes.byref(self.P), self._ws(), self._stream()))

    def plan(self) -> None:
        _lib.check(self.lib.fp_plan(ctypes.byref(self.P), self._ws(), self._stream()))

    def pool(self) -> None:
        _lib.check(self.lib.fp_pool_k(ctypes.byref(self.P), self._ws(), self._stream()))

    def search(self, dump: bool = False) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        dp = dm = None
        if dump:
            n = self.Hq * self.layout.tri_cap
            dp = torch.full((n,), float("nan"), dtype=torch.float32, device=self.device)
            dm = torch.full((n,), float("nan"), dtype=torch.float32, device=self.device)
        _lib.check(self.lib.fp_search(ctypes.byref(self.P), self._ws(),
                                      dp.data_ptr() if dump else None,
                                      dm.data_ptr() if dump else None, self._stream()))
        return (dp, dm) if dump else None

    def select(self, p_tri: torch.Tensor, m_tri: torch.Tensor) -> None:
        for t in (p_tri, m_tri):
            if t.dtype != torch.float32 or not t.is_contiguous() or \
                    t.numel() < self.Hq * self.layout.tri_cap or t.device != self.device:
                raise ValueError("scores must be contiguous fp32 device tensors of Hq*tri_cap entries")
        _lib.check(self.lib.fp_select(ctypes.byref(self.P), self._ws(), p_tri.data_ptr(),
                                      m_tri.data_ptr(), self._stream()))

    def attn(self) -> None:
        _lib.check(self.lib.fp_sparse_attn_fwd(ctypes.byref(self.P), self._ws(), self._stream()))

    def status(self) -> int:
        st = ctypes.c_uint32(0)
        _lib.check(self.lib.fp_read_status(ctypes.byref(self.P), self._ws(), self._stream(),
                                           ctypes.byref(st)))
        return int(st.value)

    # -- workspace views (valid after the stages that write them) ----------
    def _view(self, off: int, dtype: torch.dtype, n: int) -> torch.Tensor:
        nbytes = n * torch.empty((), dtype=dtype).element_size()
        return self.workspace[off:off + nbytes].view(dtype)

    def seq_tables(self) -> Tuple[List[int], List[int], List[int], List[int]]:
        L, B = self.layout, self.batch
        tile = self._view(L.seq_tile_off, torch.int64, B + 1).tolist()
        tri = self._view(L.seq_tri_off, torch.int64, B + 1).tolist()
        start = self._view(L.seq_start_off, torch.int64, B).tolist()
        ln = self._view(L.seq_len_off, torch.int32, B).tolist()
        return tile, tri, start, ln

    def items(self) -> torch.Tensor:
        tile, _, _, _ = self.seq_tables()
        return self._view(self.layout.items_off, torch.int32, 8 * tile[-1]).view(-1, 8)[:, :2]

    def sel_tables(self) -> List[int]:
        """Prefix sums of the selection blocks per sequence (the plan's block
        counts, halved and rounded up at block_size 256)."""
        tile, _, _, _ = self.seq_tables()
        out = [0]
        for b in range(self.batch):
            nb = tile[b + 1] - tile[b]
            out.append(out[-1] + (nb + self.ratio - 1) // self.ratio)
        return out

    def pooled_k(self) -> torch.Tensor:
        """Pooled K as (sum NB, Hkv, d) over the selection blocks (sequence b
        at rows sel_tables()[b] ..); the workspace holds it chunk-major
        (16-byte chunks of all key blocks of one (kv head, chunk) in a row),
        selection block j of a sequence at plan slot ratio * j."""
        tile, _, _, _ = self.seq_tables()
        cap, dt = self.layout.nb_sum_cap, self.tensors[0].dtype
        e = 16 // torch.tensor([], dtype=dt).element_size()
        raw = self._view(self.layout.mk_off, dt, self.Hkv * self.d * cap)
        slots = (raw.view(self.Hkv, self.d // e, cap, e)[:, :, :tile[-1]]
                 .permute(2, 0, 1, 3).reshape(tile[-1], self.Hkv, self.d))
        if self.ratio == 1:
            return slots
        keep = [tile[b] + j for b in range(self.batch)
                for j in range(0, tile[b + 1] - tile[b], self.ratio)]
        return slots[torch.tensor(keep, dtype=torch.long, device=slots.device)]

    def counts(self) -> torch.Tensor:
        L = self.layout
        return self._view(L.cnt_off, torch.int32, self.Hq * L.nb_sum_cap).view(self.Hq,
                                                                               L.nb_sum_cap)

    def index_lists(self) -> torch.Tensor:
        L = self.layout
        return self._view(L.idx_off, torch.int32, self.Hq * L.tri_cap).view(self.Hq, L.tri_cap)

    def _row_slots(self, b: int, tile, tri):
        """Triangular slot table of sequence b: for every (q-block i, slot n <= i)
        the flat list position tri[b] + i(i+1)/2 + n, with i and n."""
        nb = tile[b + 1] - tile[b]
        r, c = torch.tril_indices(nb, nb)
        return nb, r, c, tri[b] + r * (r + 1) // 2 + c

    def selection_masks(self) -> List[torch.Tensor]:
        """Per-sequence (Hq, NB, NB) bool masks rebuilt from the index lists (CPU)."""
        tile, tri, _, _ = self.seq_tables()
        cnt = self.counts().cpu()
        idx = self.index_lists().cpu()
        out = []
        for b in range(self.batch):
            nb, r, c, pos = self._row_slots(b, tile, tri)
            mask = torch.zeros(self.Hq, nb, nb, dtype=torch.bool)
            for h in range(self.Hq):
                valid = c < cnt[h, tile[b] + r]
                j = idx[h, pos[valid]].long()
                if j.numel() and (j.min() < 0 or j.max() >= nb):
                    raise AssertionError(f"index list entry outside [0, {nb}) in sequence {b}")
                mask[h].index_put_((r[valid], j), torch.ones((), dtype=torch.bool))
            out.append(mask)
        return out

    def ordered_lists_ok(self) -> bool:
        """True when every row's list is strictly ascending and its count is
        within the row's i + 1 slots (CPU check)."""
        tile, tri, _, _ = self.seq_tables()
        cnt = self.counts().cpu()
        idx = self.index_lists().cpu()
        for b in range(self.batch):
            nb, r, c, pos = self._row_slots(b, tile, tri)
            if nb == 0:
                continue
            rows = cnt[:, tile[b]:tile[b + 1]]
            if bool((rows < 0).any()) or bool((rows > torch.arange(1, nb + 1)).any()):
                return False
            for h in range(self.Hq):
                # consecutive valid slots n-1, n of one row must ascend
                valid = (c >= 1) & (c < cnt[h, tile[b] + r])
                p1 = pos[valid]
                if p1.numel() and not bool((idx[h, p1] > idx[h, p1 - 1]).all()):
                    return False
        return True

    def _score_slots(self, b: int, tile, tri):
        """Selection-granularity (row i, block j <= i) cells of sequence b
        and their positions in the triangular layout: row i's scores sit in
        the list slots of plan row ratio * i."""
        nb = (tile[b + 1] - tile[b] + self.ratio - 1) // self.ratio
        r, c = torch.tril_indices(nb, nb)
        pr = self.ratio * r
        return nb, r, c, tri[b] + pr * (pr + 1) // 2 + c

    def tri_scores(self, scores: Sequence[torch.Tensor]) -> torch.Tensor:
        """Pack per-sequence (Hq, NB, NB) fp32 arrays (selection blocks) into
        the triangular (Hq * tri_cap) device layout that fp_select reads."""
        tile, tri, _, _ = self.seq_tables()
        L = self.layout
        out = torch.zeros(self.Hq, L.tri_cap, dtype=torch.float32)
        for b, s in enumerate(scores):
            _, r, c, pos = self._score_slots(b, tile, tri)
            out[:, pos] = s[:, r, c].float()
        return out.reshape(-1).to(self.device)

    def untri_scores(self, flat: torch.Tensor) -> List[torch.Tensor]:
        """Inverse of tri_scores: device triangular dump -> per-sequence
        (Hq, NB, NB) CPU arrays over the selection blocks (upper triangle =
        NaN)."""
        tile, tri, _, _ = self.seq_tables()
        L = self.layout
        flat = flat.view(self.Hq, L.tri_cap).cpu()
        out = []
        for b in range(self.batch):
            nb, r, c, pos = self._score_slots(b, tile, tri)
            full = torch.full((self.Hq, nb, nb), float("nan"))
            full[:, r, c] = flat[:, pos]
            out.append(full)
        return out
