"""Device-resident spectral KV cache (three tiers) for one attention layer.

Mirrors the API of the reference ``SpectralCache`` / ``SpectralBlock``
(unsloth_spectral/spectral_cache.py:20-46, 49-704) with the storage moved
into preallocated HBM arrays managed by ``libspectral_hip.so``:

* cold tier -- INT8 coefficient codes, FP32 scales (per head, as the
  reference, or per row), FP16 bases, one slot per 512-token block;
* FP16 tail -- a ring buffer of pre-RoPE keys/values (the reference's
  hot/warm ``hot_K``/``hot_V``, grown with ``torch.cat`` at :225-227);
* per-sequence int32 counters on the device.

``append`` writes the new rows into the ring (one kernel, no concatenation)
and, when a block of ``block_size`` tokens is full, enqueues the batched rSVD
compressor for every full block (no host round-trip: the host knows how many
tokens it appended, so it knows when a block fills).  Like the reference,
compression fires as soon as the tail reaches ``block_size`` (:238).

A cache holds ``batch`` independent sequences (the reference holds one and
asserts batch 1 at :346); all sequences are appended together.
"""
import copy
import ctypes
import math
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

from . import _lib
from ._lib import check, ptr


@dataclass
class SpectralBlock:
    """One compressed block (spectral_cache.py:20-46).

    ``coeffs_*`` are the dequantised coefficients fp16(code*scale) (what the
    reference stores), ``scales_*`` the reference's per-head [min, max]."""
    coeffs_K: torch.Tensor
    basis_K: torch.Tensor
    coeffs_V: torch.Tensor
    basis_V: torch.Tensor
    scales_K: torch.Tensor
    scales_V: torch.Tensor
    block_size: int
    start_position: int


def _first_position(position_ids, T):
    """The first new position as a host integer, for the new-generation test
    (spectral_cache.py:177-189), or None when reading it would cost a
    device-to-host synchronisation on the decode path.

    Host data (ints, sequences, numpy arrays, CPU tensors) is read directly.
    A device tensor is read only for a multi-token append (prompt prefill or
    a chunk of it, where the reference reads it too); a one-token append
    with device positions is taken to continue the sequence, so a decode
    step never waits for the device.  A new generation that starts with a
    one-token prompt is therefore detected only from host positions or by
    calling ``reset()`` first."""
    if isinstance(position_ids, int):
        return position_ids
    if isinstance(position_ids, torch.Tensor):
        if position_ids.numel() == 0:
            return None
        if position_ids.device.type != "cpu" and T <= 1:
            return None
        return int(position_ids.reshape(-1)[0])
    try:
        import numpy as np
        arr = np.asarray(position_ids).reshape(-1)
        return int(arr[0]) if arr.size else None
    except (TypeError, ValueError):
        return None


def padded_rank(k):
    """Storage rank of the INT8 codes / bases (zero-padded)."""
    for kp in (16, 32, 64):
        if k <= kp:
            return kp
    raise ValueError(f"rank {k} > 64 is not supported by the HIP kernels")


class SpectralCache:
    """Three-tier KV cache with automatic spectral compression.

    Arguments follow spectral_cache.py:72-87; keyword-only extras:
      batch_size        sequences held (default: taken from the first append)
      max_blocks        initial cold capacity per sequence (grows on demand)
      tail_capacity     initial FP16 ring capacity (grows on demand)
      quant_granularity "per_head" (reference) or "per_row"
      oversampling, n_iter   rSVD parameters (rsvd.py defaults 5, 2)
      seed              seed of the on-device Gaussian sketch
    ``hot_buffer_size`` is stored but unused, as in the reference (:93).
    ``use_attention_weighted_svd`` and landmarks behave as in the reference:
    the block compression of ``append`` never passes attention weights
    (:285-286), and landmark tokens enter only through ``add_landmarks``;
    ``_compress_tensor``, ``update_attention_importance``,
    ``get_block_attention_weights``, ``add_landmarks`` and
    ``get_kv_with_landmarks`` are the reference's (:321-407, :710-852)."""

    def __init__(self, num_heads: int, head_dim: int, block_size: int = 512, k_rank_keys: int = 16,
                 k_rank_values: int = 32, hot_buffer_size: int = 64, device="cuda",
                 dtype: torch.dtype = torch.float16, debug_logging: bool = False,
                 use_attention_weighted_svd: bool = False, landmark_positions: Optional[List[int]] = None,
                 landmark_count: int = 0, *, batch_size: Optional[int] = None, max_blocks: Optional[int] = None,
                 tail_capacity: Optional[int] = None, quant_granularity: str = "per_head",
                 oversampling: int = 5, n_iter: int = 2, seed: int = 0):
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("SpectralCache stores its tiers in GPU memory; device must be a ROCm device "
                               f"(got {device})")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        if dtype != torch.float16:
            raise NotImplementedError("the HIP tiers hold float16 keys/values (got %s)" % dtype)
        if quant_granularity not in ("per_head", "per_row"):
            raise ValueError("quant_granularity must be 'per_head' or 'per_row'")
        if block_size % 64 or block_size <= 0:
            raise ValueError("block_size must be a positive multiple of 64")
        _lib.load()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.k_rank_keys = k_rank_keys
        self.k_rank_values = k_rank_values
        self.hot_buffer_size = hot_buffer_size
        self.device = device
        self.dtype = dtype
        self.debug_logging = debug_logging
        self.use_attention_weighted_svd = use_attention_weighted_svd
        self.landmark_positions = set(landmark_positions) if landmark_positions else set()
        self.landmark_count = landmark_count
        self.quant_granularity = quant_granularity
        self.oversampling = oversampling
        self.n_iter = n_iter
        self.seed = seed
        self.kp_keys = padded_rank(k_rank_keys)
        self.kp_values = padded_rank(k_rank_values)
        self.cache_id = id(self)
        self._max_blocks = max(1, max_blocks or 8)
        self._tail_cap = max(2 * block_size, tail_capacity or 0)
        self._B = None
        self._desc = None
        self._compress_calls = 0
        if batch_size is not None:
            self._allocate(batch_size)
        self._zero_host()

    # ------------------------------------------------------------ storage
    def _zero_host(self):
        self.attention_importance = None
        self.landmark_K = None
        self.landmark_V = None
        self.landmark_position_ids = None
        self.total_tokens = 0
        self.current_position = 0
        self.compression_count = 0
        self._n_cold = 0
        self._tail_len = 0
        self._tail_head = 0
        self.key_mask = None
        # Decode grid pinned for a captured (graph-replayed) decode segment:
        # the decode launch covers this many tail tokens whatever the host
        # mirror says (None = the mirror's tail length).
        self._grid_tail = None

    def _allocate(self, batch):
        B, H, D, TB, NB, C = batch, self.num_heads, self.head_dim, self.block_size, self._max_blocks, self._tail_cap
        dev = self.device
        per_row = self.quant_granularity == "per_row"
        self._B = B
        self.codes_k = torch.zeros(B, H, NB, TB, self.kp_keys, dtype=torch.int8, device=dev)
        self.codes_v = torch.zeros(B, H, NB, self.kp_values, TB, dtype=torch.int8, device=dev)
        sshape = (B, H, NB, TB) if per_row else (B, H, NB)
        self.scales_k = torch.ones(sshape, dtype=torch.float32, device=dev)
        self.scales_v = torch.ones(sshape, dtype=torch.float32, device=dev)
        self.minmax_k = torch.zeros(B, H, NB, 2, dtype=torch.float32, device=dev)
        self.minmax_v = torch.zeros(B, H, NB, 2, dtype=torch.float32, device=dev)
        self.vnorm = torch.ones(B, H, NB, dtype=torch.float32, device=dev)
        self.basis_k = torch.zeros(B, H, NB, D, self.kp_keys, dtype=torch.float16, device=dev)
        self.basis_v = torch.zeros(B, H, NB, D, self.kp_values, dtype=torch.float16, device=dev)
        self.block_start = torch.zeros(B, NB, dtype=torch.int32, device=dev)
        self.tail_k = torch.zeros(B, H, C, D, dtype=torch.float16, device=dev)
        self.tail_v = torch.zeros(B, H, C, D, dtype=torch.float16, device=dev)
        self.tail_pos = torch.zeros(B, C, dtype=torch.int32, device=dev)
        self.counters = torch.zeros(B, _lib.SC_NCOUNTERS, dtype=torch.int32, device=dev)
        self._desc = None

    def _tier(self):
        """ctypes descriptor of the current buffers (rebuilt after growth)."""
        if self._desc is None:
            d = _lib.ScTierDesc()
            d.batch, d.kv_heads, d.head_dim, d.block_size = self._B, self.num_heads, self.head_dim, self.block_size
            d.k_keys, d.k_values = self.k_rank_keys, self.k_rank_values
            d.kp_keys, d.kp_values = self.kp_keys, self.kp_values
            d.max_blocks, d.tail_capacity = self._max_blocks, self._tail_cap
            d.granularity = _lib.GRANULARITY[self.quant_granularity]
            for name in ("codes_k", "codes_v", "scales_k", "scales_v", "minmax_k", "minmax_v", "vnorm",
                         "basis_k", "basis_v", "block_start", "tail_k", "tail_v", "tail_pos", "counters"):
                setattr(d, name, getattr(self, name).data_ptr())
            self._desc = d
            self._desc_ptr = ctypes.pointer(d)
        return self._desc

    def _tier_ptr(self):
        """ctypes pointer to the current descriptor (kept with it)."""
        self._tier()
        return self._desc_ptr

    def _grow_cold(self, need):
        if need <= self._max_blocks:
            return
        nb = self._max_blocks
        while nb < need:
            nb *= 2
        old = {n: getattr(self, n) for n in ("codes_k", "codes_v", "scales_k", "scales_v", "minmax_k",
                                              "minmax_v", "vnorm", "basis_k", "basis_v", "block_start")}
        tail = {n: getattr(self, n) for n in ("tail_k", "tail_v", "tail_pos", "counters")}
        self._max_blocks = nb
        self._allocate(self._B)
        for n, t in old.items():
            dst = getattr(self, n)
            if n == "block_start":
                dst[:, :t.shape[1]].copy_(t)
            else:
                dst[:, :, :t.shape[2]].copy_(t)
        for n, t in tail.items():
            setattr(self, n, t)
        self._desc = None

    def _grow_tail(self, need):
        if need <= self._tail_cap:
            return
        cap = self._tail_cap
        while cap < need:
            cap *= 2
        idx = (self._tail_head + torch.arange(self._tail_len, device=self.device)) % self._tail_cap
        tk = torch.zeros(self._B, self.num_heads, cap, self.head_dim, dtype=torch.float16, device=self.device)
        tv = torch.zeros_like(tk)
        tp = torch.zeros(self._B, cap, dtype=torch.int32, device=self.device)
        if self._tail_len:
            tk[:, :, :self._tail_len] = self.tail_k.index_select(2, idx)
            tv[:, :, :self._tail_len] = self.tail_v.index_select(2, idx)
            tp[:, :self._tail_len] = self.tail_pos.index_select(1, idx)
        self.tail_k, self.tail_v, self.tail_pos = tk, tv, tp
        self.counters[:, _lib.SC_CNT_TAIL_HEAD] = 0
        self._tail_head = 0
        self._tail_cap = cap
        self._desc = None

    def reserve(self, tokens: int, batch_size: Optional[int] = None):
        """Sizes the tiers for ``tokens`` tokens per sequence (cold slots for
        every full block, a ring of at least two blocks), so that appends up
        to that length allocate nothing: a decode step then neither allocates
        nor waits for the device.  ``batch_size`` allocates a cache that has
        not seen an append yet."""
        if self._B is None:
            if batch_size is None:
                raise ValueError("reserve() on an empty cache needs batch_size")
            self._max_blocks = max(self._max_blocks, tokens // self.block_size)
            self._allocate(batch_size)
            return
        self._grow_cold(tokens // self.block_size)

    _BUFFERS = ("codes_k", "codes_v", "scales_k", "scales_v", "minmax_k", "minmax_v", "vnorm", "basis_k",
                "basis_v", "block_start", "tail_k", "tail_v", "tail_pos", "counters")

    def clone(self):
        """Deep copy (new device buffers, same tiers and counters)."""
        c = copy.copy(self)
        if self._B is not None:
            for name in self._BUFFERS:
                setattr(c, name, getattr(self, name).clone())
        if self.key_mask is not None:
            c.key_mask = self.key_mask.clone()
        c._desc = None
        c.cache_id = id(c)
        return c

    # ------------------------------------------------------------ reference API
    def reset(self):
        """spectral_cache.py:137-162"""
        if self._B is not None:
            self.counters.zero_()
        self._zero_host()

    def append(self, K_new: torch.Tensor, V_new: torch.Tensor, position_ids: Optional[torch.Tensor] = None):
        """spectral_cache.py:164-241: K_new, V_new [B, H, T_new, D] (pre-RoPE)."""
        _lib.require_device(K_new, "K_new")
        if K_new.dim() != 4 or K_new.shape != V_new.shape:
            raise ValueError(f"K_new/V_new must be [B, H, T, D] of equal shape, got {tuple(K_new.shape)} "
                             f"and {tuple(V_new.shape)}")
        B, H, T, D = K_new.shape
        if H != self.num_heads or D != self.head_dim:
            raise ValueError(f"expected {self.num_heads} heads of dim {self.head_dim}, got {H} x {D}")
        if self._B is None:
            self._allocate(B)
        elif B != self._B:
            raise ValueError(f"cache holds {self._B} sequences, append has {B}")
        flags = 0
        if position_ids is not None and self.total_tokens > 0:
            first = _first_position(position_ids, T)          # :177-183
            if first is not None and first < self.current_position:
                self._zero_host()                              # :186-189; counters cleared by the append kernel
                flags = _lib.SC_APPEND_RESET
        if T == 0:
            if flags:
                self.counters.zero_()
            return
        K16 = K_new if K_new.dtype == torch.float16 else K_new.to(torch.float16)
        V16 = V_new if V_new.dtype == torch.float16 else V_new.to(torch.float16)
        if K16.stride(-1) != 1 or K16.stride(2) % 8 or K16.stride(1) % 8 or K16.stride(0) % 8 or \
                K16.data_ptr() % 16:
            K16 = K16.contiguous()
        if V16.stride() != K16.stride() or V16.data_ptr() % 16:
            V16 = V16.contiguous()
            K16 = K16.contiguous()
        pos = None
        if position_ids is not None:
            if not isinstance(position_ids, torch.Tensor):
                position_ids = torch.as_tensor(position_ids)
            pos = position_ids.reshape(-1, T)
            if pos.dtype == torch.int64 and pos.device == self.device and pos.shape[0] == B and \
                    pos.is_contiguous():
                flags |= _lib.SC_APPEND_POS_I64     # a model's position ids as they are (no conversion launch)
            else:
                pos = pos.to(device=self.device, dtype=torch.int32)
                pos = pos.expand(B, T).contiguous() if pos.shape[0] != B else pos.contiguous()
        self._grow_tail(self._tail_len + T)
        st = _lib.stream_of(K16)
        check(_lib.load().sc_tier_append(self._tier_ptr(), ptr(K16), ptr(V16), K16.stride(0),
                                         K16.stride(1), K16.stride(2), ptr(pos), T, flags, st))
        self.total_tokens += T
        self.current_position += T
        self._tail_len += T
        if self._tail_len >= self.block_size:               # :238-241
            self._compress_hot_cache()

    def _compress_hot_cache(self):
        """spectral_cache.py:243-319 -- every full block, one batched launch."""
        nfull = self._tail_len // self.block_size
        if nfull == 0:
            return
        self._grow_cold(self._n_cold + nfull)
        st = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        seed = (self.seed * 0x9E3779B97F4A7C15 + self._compress_calls) & 0xFFFFFFFFFFFFFFFF
        self._compress_calls += 1
        check(_lib.load().sc_tier_compress(ctypes.byref(self._tier()), nfull, self.n_iter, self.oversampling,
                                           seed, st))
        self._n_cold += nfull
        self._tail_head = (self._tail_head + nfull * self.block_size) % self._tail_cap
        self._tail_len -= nfull * self.block_size
        self.compression_count += nfull

    # ------------------------------------------------------------ views
    @property
    def num_cold_blocks(self):
        return self._n_cold

    @property
    def hot_len(self):
        return self._tail_len

    def _tail_index(self):
        return (self._tail_head + torch.arange(self._tail_len, device=self.device)) % self._tail_cap

    @property
    def hot_K(self):
        if self._B is None or self._tail_len == 0:
            return None
        return self.tail_k.index_select(2, self._tail_index())

    @property
    def hot_V(self):
        if self._B is None or self._tail_len == 0:
            return None
        return self.tail_v.index_select(2, self._tail_index())

    @property
    def hot_position_ids(self):
        if self._B is None or self._tail_len == 0:
            return None
        return self.tail_pos.index_select(1, self._tail_index()).to(torch.long)

    def _dequant_coeffs(self, j, kind):
        if kind == "K":
            codes = self.codes_k[:, :, j, :, :self.k_rank_keys].float()
            sc = self.scales_k[:, :, j]
        else:
            codes = self.codes_v[:, :, j, :self.k_rank_values, :].transpose(-1, -2).float()
            sc = self.scales_v[:, :, j]
        sc = sc.unsqueeze(-1) if sc.dim() == 3 else sc.reshape(sc.shape + (1, 1))
        return (codes * sc).to(torch.float16)

    @property
    def cold_blocks(self) -> List[SpectralBlock]:
        out = []
        if self._B is None or self._n_cold == 0:
            return out
        starts = self.block_start[0, :self._n_cold].tolist()
        squeeze = self._B == 1
        for j in range(self._n_cold):
            ck = self._dequant_coeffs(j, "K")
            cv = self._dequant_coeffs(j, "V")
            bk = self.basis_k[:, :, j, :, :self.k_rank_keys].transpose(-1, -2).contiguous()
            bv = self.basis_v[:, :, j, :, :self.k_rank_values].transpose(-1, -2).contiguous()
            mk, mv = self.minmax_k[:, :, j], self.minmax_v[:, :, j]
            if squeeze:
                ck, cv, bk, bv, mk, mv = ck[0], cv[0], bk[0], bv[0], mk[0], mv[0]
            out.append(SpectralBlock(ck, bk, cv, bv, mk, mv, self.block_size, int(starts[j])))
        return out

    def get_spectral_components(self) -> Tuple[List[SpectralBlock], Optional[torch.Tensor], Optional[torch.Tensor]]:
        """spectral_cache.py:518-527"""
        return self.cold_blocks, self.hot_K, self.hot_V

    def positions(self) -> torch.Tensor:
        """Positions of every cached token of every sequence, [B, L] int64
        in cache order (cold blocks, then the tail oldest first)."""
        if self._B is None:
            return torch.empty(0, 0, dtype=torch.long, device=self.device)
        parts = []
        if self._n_cold:
            ar = torch.arange(self.block_size, device=self.device)
            parts.append((self.block_start[:, :self._n_cold, None].to(torch.long) + ar).reshape(self._B, -1))
        if self._tail_len:
            parts.append(self.tail_pos.index_select(1, self._tail_index()).to(torch.long))
        if not parts:
            return torch.empty(self._B, 0, dtype=torch.long, device=self.device)
        return torch.cat(parts, dim=1)

    # ------------------------------------------------------------ padding (key keep-mask)
    # Batched generation with left padding: the prompt's pad tokens are
    # appended like the others, so the cache keeps one keep flag per cached
    # token (uint8 [B, capacity], 1 = attend) once a padding mask has been
    # recorded; decode calls pass it as their keep-mask.  The reference's
    # cache holds one sequence and has no such state.
    def record_key_mask(self, keep: torch.Tensor, start: int):
        """Keep flags [B, T] of the tokens at cache indices start .. start+T-1."""
        T = keep.shape[-1]
        need = start + T
        km = self.key_mask
        if km is None or km.shape[1] < need:
            cap = max(need, 2 * (km.shape[1] if km is not None else self.block_size))
            new = torch.ones(self._B, cap, dtype=torch.uint8, device=self.device)
            if km is not None:
                new[:, :km.shape[1]] = km
            self.key_mask = km = new
        km[:, start:need] = keep.to(torch.uint8)

    def key_mask_view(self) -> Optional[torch.Tensor]:
        """[B, total] keep flags of the cached tokens, or None without padding."""
        if self.key_mask is None:
            return None
        n = self._n_cold * self.block_size + self._tail_len
        if self.key_mask.shape[1] < n:
            self.record_key_mask(torch.ones(self._B, n - self.key_mask.shape[1], dtype=torch.uint8,
                                            device=self.device), self.key_mask.shape[1])
        return self.key_mask[:, :n]

    def get_all_positions(self) -> torch.Tensor:
        """spectral_cache.py:529-555 (sequence 0)."""
        parts = []
        if self._B is not None:
            for s in self.block_start[0, :self._n_cold].tolist():
                parts.append(torch.arange(s, s + self.block_size, device=self.device, dtype=torch.long))
            hp = self.hot_position_ids
            if hp is not None:
                parts.append(hp[0])
        if not parts:
            return torch.empty(0, device=self.device, dtype=torch.long)
        return torch.cat(parts)

    def get_kv(self):
        """spectral_cache.py:557-612: fp16 reconstruction [B, H, T, D] (None, None if empty)."""
        if self._B is None or self.total_tokens == 0 or (self._n_cold == 0 and self._tail_len == 0):
            return None, None
        parts_k, parts_v = [], []
        if self._n_cold:
            shape = (self._B, self.num_heads, self._n_cold * self.block_size, self.head_dim)
            k = torch.empty(shape, dtype=torch.float16, device=self.device)
            v = torch.empty_like(k)
            check(_lib.load().sc_tier_dequant(ctypes.byref(self._tier()), 0, self._n_cold, ptr(k), ptr(v),
                                              _lib.stream_of(k)))
            parts_k.append(k)
            parts_v.append(v)
        if self._tail_len:
            parts_k.append(self.hot_K)
            parts_v.append(self.hot_V)
        return torch.cat(parts_k, dim=2), torch.cat(parts_v, dim=2)

    # ------------------------------------------------------------ weighted SVD, landmarks
    def _compress_tensor(self, X: torch.Tensor, rank: int, attention_weights: Optional[torch.Tensor] = None):
        """spectral_cache.py:321-407: compresses X [1, H, T, D] on the device.

        Returns (coeffs [H, T, rank] = dequantised INT8 codes in the cache
        dtype, basis [H, rank, D] in the cache dtype, scales [H, 2] = per-head
        (min, max) of the coefficients).  With ``use_attention_weighted_svd``
        and ``attention_weights`` [T], rows are weighted by
        sqrt(a / mean(a)) for the SVD and the coefficients unweighted
        (:351-368, :389-393).  The Gaussian sketch is drawn on the device."""
        from .rsvd import compress_matrices
        _lib.require_device(X, "X")
        B, H, T, D = X.shape
        if B != 1:
            raise ValueError("Batch size must be 1 for now")   # :346
        M = X[0]
        if M.dtype not in _lib.SC_DTYPE:
            M = M.float()
        w = None
        if self.use_attention_weighted_svd and attention_weights is not None:
            w = attention_weights.reshape(-1)
            if w.numel() != T:
                raise ValueError(f"attention_weights must hold {T} entries, got {w.numel()}")
        seed = (self.seed * 0x9E3779B97F4A7C15 + self._compress_calls) & 0xFFFFFFFFFFFFFFFF
        self._compress_calls += 1
        res = compress_matrices(M, rank, self.n_iter, self.oversampling, seed=seed, granularity="per_head",
                                row_weights=w)
        kp_codes = res["codes"][:, :, :rank].float()
        coeffs = (kp_codes * res["scales"][:, None, None]).to(self.dtype)
        basis = res["basis"][:, :rank, :].to(self.dtype)
        return coeffs, basis, res["minmax"]

    def update_attention_importance(self, attention_weights: torch.Tensor, query_position: int):
        """spectral_cache.py:710-750: running average (alpha 0.1) of the
        attention probabilities [B, H, 1, T_kv] averaged over batch and
        heads; no-op unless ``use_attention_weighted_svd``."""
        if not self.use_attention_weighted_svd:
            return
        avg = attention_weights.mean(dim=(0, 1, 2))
        if self.attention_importance is None:
            self.attention_importance = avg.clone()
            return
        alpha = 0.1
        if self.attention_importance.shape[0] < avg.shape[0]:
            pad = torch.zeros(avg.shape[0] - self.attention_importance.shape[0], device=avg.device, dtype=avg.dtype)
            self.attention_importance = torch.cat([self.attention_importance, pad])
        n = avg.shape[0]
        self.attention_importance[:n] = (1 - alpha) * self.attention_importance[:n] + alpha * avg

    def get_block_attention_weights(self, block_idx: int) -> Optional[torch.Tensor]:
        """spectral_cache.py:752-777: importance of block ``block_idx``'s
        tokens, or None when not tracked that far."""
        if self.attention_importance is None:
            return None
        start = block_idx * self.block_size
        end = start + self.block_size
        if end > self.attention_importance.shape[0]:
            return None
        return self.attention_importance[start:end]

    def add_landmarks(self, K: torch.Tensor, V: torch.Tensor, position_ids: torch.Tensor):
        """spectral_cache.py:779-802: FP16 tokens that are never compressed,
        K, V [B, H, T, D], position_ids [B, T]; appended to earlier ones."""
        _lib.require_device(K, "K")
        if self.landmark_K is None:
            self.landmark_K = K.clone()
            self.landmark_V = V.clone()
            self.landmark_position_ids = position_ids.clone()
        else:
            self.landmark_K = torch.cat([self.landmark_K, K], dim=2)
            self.landmark_V = torch.cat([self.landmark_V, V], dim=2)
            self.landmark_position_ids = torch.cat([self.landmark_position_ids, position_ids], dim=1)

    def get_kv_with_landmarks(self):
        """spectral_cache.py:804-852: (K, V, position_ids) with landmarks
        first, then the reconstructed cold blocks, then the FP16 tail;
        (None, None, None) when everything is empty."""
        K_parts, V_parts, pos_parts = [], [], []
        if self.landmark_K is not None:
            K_parts.append(self.landmark_K)
            V_parts.append(self.landmark_V)
            if self.landmark_position_ids is not None:
                pos_parts.append(self.landmark_position_ids)
        if self._B is not None and self.total_tokens > 0 and self._n_cold:
            shape = (self._B, self.num_heads, self._n_cold * self.block_size, self.head_dim)
            k = torch.empty(shape, dtype=torch.float16, device=self.device)
            v = torch.empty_like(k)
            check(_lib.load().sc_tier_dequant(ctypes.byref(self._tier()), 0, self._n_cold, ptr(k), ptr(v),
                                              _lib.stream_of(k)))
            K_parts.append(k)
            V_parts.append(v)
            ar = torch.arange(self.block_size, device=self.device)
            for j in range(self._n_cold):  # [B, T] positions of block j of every sequence
                pos_parts.append(self.block_start[:, j:j + 1].to(torch.long) + ar)
        if self._B is not None and self.total_tokens > 0 and self._tail_len:
            K_parts.append(self.hot_K)
            V_parts.append(self.hot_V)
            hp = self.hot_position_ids
            if hp is not None:
                pos_parts.append(hp)
        if not K_parts:
            return None, None, None
        dt = K_parts[0].dtype
        K_full = torch.cat([x.to(dt) for x in K_parts], dim=2)
        V_full = torch.cat([x.to(dt) for x in V_parts], dim=2)
        pos = torch.cat([p_.to(torch.long) for p_ in pos_parts], dim=1) if pos_parts else None
        return K_full, V_full, pos

    def get_memory_stats(self) -> dict:
        """spectral_cache.py:614-655 with the bytes this cache actually stores."""
        B = self._B or 1
        H = self.num_heads
        original = self.total_tokens * H * self.head_dim * 2 * 2 * B
        per_row = self.quant_granularity == "per_row"
        nb = self._n_cold
        comp = B * H * nb * (self.block_size * (self.kp_keys + self.kp_values)
                             + self.head_dim * (self.kp_keys + self.kp_values) * 2
                             + (2 * self.block_size * 4 if per_row else 2 * 4) + 4 * 4)
        comp += B * H * self._tail_len * self.head_dim * 2 * 2
        return {
            "original_bytes": original,
            "compressed_bytes": comp,
            "compression_ratio": original / comp if comp > 0 else 1.0,
            "num_blocks": nb,
            "total_tokens": self.total_tokens,
        }

    def __len__(self):
        return self.total_tokens

    def __getitem__(self, index):
        """spectral_cache.py:661-686 (tuple emulation for Unsloth)."""
        if index == 0:
            return self.get_kv()[0]
        if index == 1:
            return self.get_kv()[1]
        raise IndexError(f"SpectralCache subscript index out of range: {index} (expected 0 or 1)")

    def __iter__(self):
        K, V = self.get_kv()
        yield K
        yield V

    def __repr__(self):
        s = self.get_memory_stats()
        return (f"SpectralCache(tokens={self.total_tokens}, blocks={s['num_blocks']}, "
                f"compression={s['compression_ratio']:.2f}x)")

    # ------------------------------------------------------------ wire format
    # No counterpart in the reference (its blocks are Python objects,
    # spectral_cache.py:20-46); records: unsloth_spectral.wire.
    def block_record_bytes(self) -> int:
        """Bytes of one cold-block record of this cache's geometry."""
        d = _lib.ScTierDesc()
        d.batch, d.kv_heads, d.head_dim, d.block_size = 1, self.num_heads, self.head_dim, self.block_size
        d.k_keys, d.k_values, d.kp_keys, d.kp_values = self.k_rank_keys, self.k_rank_values, self.kp_keys, \
            self.kp_values
        d.granularity = _lib.GRANULARITY[self.quant_granularity]
        return int(_lib.load().sc_block_record_bytes(ctypes.byref(d)))

    def export_blocks(self, seq: int = 0, first: int = 0, count: Optional[int] = None) -> torch.Tensor:
        """Cold blocks [first, first + count) of sequence ``seq`` packed into
        consecutive records (uint8 device tensor) by sc_tier_pack; count
        defaults to every block from ``first`` on."""
        rb = self.block_record_bytes()
        n = (self._n_cold - first) if count is None else count
        if self._B is None or n <= 0:
            return torch.empty(0, dtype=torch.uint8, device=self.device)
        if not 0 <= seq < self._B or first < 0 or first + n > self._n_cold:
            raise ValueError(f"blocks [{first}, {first + n}) of sequence {seq} are not all in use "
                             f"({self._n_cold} cold blocks, {self._B} sequences)")
        out = torch.empty(n * rb, dtype=torch.uint8, device=self.device)
        st = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        check(_lib.load().sc_tier_pack(ctypes.byref(self._tier()), seq, first, n, ptr(out), out.numel(), st))
        return out

    def import_blocks(self, records: torch.Tensor, seq: int = 0, first: Optional[int] = None) -> int:
        """Unpacks block records (uint8 tensor, host or device) into cold
        slots first, first + 1, ... of sequence ``seq`` (default: after the
        blocks in use) by sc_tier_unpack; returns the number of blocks.
        If any record's header does not match this cache's geometry
        (checked on the device) nothing is written and SpectralHIPError is
        raised."""
        if self._B is None:
            raise ValueError("the cache holds no sequences yet (append or construct with batch_size)")
        rb = self.block_record_bytes()
        if records.dtype != torch.uint8 or records.dim() != 1 or records.numel() % rb:
            raise ValueError(f"records must be a flat uint8 tensor of whole {rb}-byte records")
        n = records.numel() // rb
        if not 0 <= seq < self._B:
            raise ValueError(f"sequence {seq} outside [0, {self._B})")
        first = self._n_cold if first is None else first
        if n == 0:
            return 0
        self._grow_cold(first + n)
        buf = records.to(self.device)
        if buf.data_ptr() % 16:
            buf = buf.clone()
        status = torch.zeros(1, dtype=torch.int32, device=self.device)
        st = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        check(_lib.load().sc_tier_unpack(ctypes.byref(self._tier()), seq, first, n, ptr(buf), buf.numel(),
                                         ptr(status), st))
        code = int(status.item())
        if code:
            raise _lib.SpectralHIPError(f"block records do not match this cache's geometry (code {code}); "
                                        "none were taken")
        self._n_cold = max(self._n_cold, first + n)
        return n

    def save(self, path: str):
        """Writes the cache (every sequence's cold blocks as records, the FP16
        tails and the counters) to a safetensors file."""
        import json
        from safetensors.torch import save_file
        if self._B is None:
            raise ValueError("nothing to save: the cache holds no sequences")
        ncold = self.counters[:, _lib.SC_CNT_NCOLD].tolist()
        tensors = {"counters": self.counters.cpu(), "tail_k": self.tail_k.cpu(), "tail_v": self.tail_v.cpu(),
                   "tail_pos": self.tail_pos.cpu()}
        for b in range(self._B):
            tensors[f"blocks.{b}"] = self.export_blocks(b, 0, ncold[b]).cpu()
        meta = {"num_heads": self.num_heads, "head_dim": self.head_dim, "block_size": self.block_size,
                "k_rank_keys": self.k_rank_keys, "k_rank_values": self.k_rank_values,
                "hot_buffer_size": self.hot_buffer_size, "quant_granularity": self.quant_granularity,
                "oversampling": self.oversampling, "n_iter": self.n_iter, "seed": self.seed,
                "batch": self._B, "tail_capacity": self._tail_cap, "n_cold": self._n_cold,
                "tail_len": self._tail_len, "tail_head": self._tail_head, "total_tokens": self.total_tokens,
                "current_position": self.current_position, "compression_count": self.compression_count,
                "compress_calls": self._compress_calls}
        save_file(tensors, path, metadata={"format": "spectral-cache/1", "cache": json.dumps(meta)})

    @classmethod
    def load(cls, path: str, device="cuda") -> "SpectralCache":
        """Reads a file written by save()."""
        import json
        from safetensors import safe_open
        with safe_open(path, framework="pt") as f:
            meta = f.metadata() or {}
            if meta.get("format") != "spectral-cache/1":
                raise ValueError(f"{path} is not a saved SpectralCache")
            m = json.loads(meta["cache"])
            tensors = {k: f.get_tensor(k) for k in f.keys()}
        c = cls(m["num_heads"], m["head_dim"], block_size=m["block_size"], k_rank_keys=m["k_rank_keys"],
                k_rank_values=m["k_rank_values"], hot_buffer_size=m["hot_buffer_size"], device=device,
                batch_size=m["batch"], max_blocks=max(1, m["n_cold"]), tail_capacity=m["tail_capacity"],
                quant_granularity=m["quant_granularity"], oversampling=m["oversampling"], n_iter=m["n_iter"],
                seed=m["seed"])
        for b in range(m["batch"]):
            c.import_blocks(tensors[f"blocks.{b}"], seq=b, first=0)
        c.tail_k.copy_(tensors["tail_k"])
        c.tail_v.copy_(tensors["tail_v"])
        c.tail_pos.copy_(tensors["tail_pos"])
        c.counters.copy_(tensors["counters"])
        c._n_cold, c._tail_len, c._tail_head = m["n_cold"], m["tail_len"], m["tail_head"]
        c.total_tokens, c.current_position = m["total_tokens"], m["current_position"]
        c.compression_count, c._compress_calls = m["compression_count"], m["compress_calls"]
        return c

    # ------------------------------------------------------------ construction from explicit tiers
    @classmethod
    def from_tiers(cls, codes_k, scales_k, basis_k, codes_v, scales_v, basis_v, block_start,
                   tail_k=None, tail_v=None, tail_pos=None, *, block_size=None, tail_capacity=None,
                   minmax_k=None, minmax_v=None, seed=0, max_blocks=None):
        """Builds a cache from explicit tiers (the reference builds tier states
        only by appending; configs with a 448+64-token tail need them built
        directly).  Layouts (B sequences, H KV heads, NB blocks, T tokens):
          codes_k/v  int8 [B, H, NB, T, k]     scales_k/v  f32 [B, H, NB] or [B, H, NB, T]
          basis_k/v  f16  [B, H, NB, k, D]     block_start int [B, NB]
          tail_k/v   f16  [B, H, Tt, D] (pre-RoPE)   tail_pos int [B, Tt]
        ``max_blocks`` reserves cold-tier room beyond NB (later compressions
        then reuse it instead of growing the tier buffers)."""
        B, H, NB, T, kK = codes_k.shape
        kV = codes_v.shape[-1]
        D = basis_k.shape[-1]
        per_row = scales_k.dim() == 4
        Tt = 0 if tail_k is None else tail_k.shape[2]
        cap = max(tail_capacity or 0, 2 * (block_size or T), Tt)
        c = cls(H, D, block_size=block_size or T, k_rank_keys=kK, k_rank_values=kV, device=codes_k.device,
                batch_size=B, max_blocks=max(NB, 1, max_blocks or 0), tail_capacity=cap,
                quant_granularity="per_row" if per_row else "per_head", seed=seed)
        if NB:
            c.codes_k[:, :, :NB, :, :kK] = codes_k
            c.codes_v[:, :, :NB, :kV, :] = codes_v.transpose(-1, -2)
            c.scales_k[:, :, :NB] = scales_k
            c.scales_v[:, :, :NB] = scales_v
            c.basis_k[:, :, :NB, :, :kK] = basis_k.transpose(-1, -2).to(torch.float16)
            c.basis_v[:, :, :NB, :, :kV] = basis_v.transpose(-1, -2).to(torch.float16)
            c.block_start[:, :NB] = block_start.to(torch.int32)
            vmax = scales_v.reshape(B, H, NB, -1).amax(-1)
            _, e = torch.frexp(vmax)
            c.vnorm[:, :, :NB] = torch.ldexp(torch.ones_like(vmax), -e)
            for name, given, codes, sc in (("minmax_k", minmax_k, codes_k, scales_k),
                                           ("minmax_v", minmax_v, codes_v, scales_v)):
                if given is None:
                    deq = codes.float() * (sc.unsqueeze(-1) if per_row else sc.reshape(B, H, NB, 1, 1))
                    given = torch.stack([deq.amin(dim=(-1, -2)), deq.amax(dim=(-1, -2))], -1)
                getattr(c, name)[:, :, :NB] = given
        if Tt:
            c.tail_k[:, :, :Tt] = tail_k
            c.tail_v[:, :, :Tt] = tail_v
            c.tail_pos[:, :Tt] = tail_pos.to(torch.int32)
        cnt = torch.zeros(B, _lib.SC_NCOUNTERS, dtype=torch.int32)
        cnt[:, _lib.SC_CNT_NCOLD] = NB
        cnt[:, _lib.SC_CNT_TAIL_LEN] = Tt
        cnt[:, _lib.SC_CNT_NEXT_POS] = NB * T + Tt
        cnt[:, _lib.SC_CNT_TOTAL] = NB * T + Tt
        cnt[:, _lib.SC_CNT_COMPRESSIONS] = NB
        c.counters.copy_(cnt)
        c._n_cold, c._tail_len, c._tail_head = NB, Tt, 0
        c.total_tokens = c.current_position = NB * T + Tt
        c.compression_count = NB
        return c

    @classmethod
    def from_components(cls, cold_blocks, hot_K, hot_V, hot_position_ids, num_heads=None, device=None):
        """Imports a reference-style cache (list of SpectralBlock with
        dequantised fp16 coefficients and per-head [min, max]).  INT8 codes are
        recovered exactly: scale = max(|min|, |max|, 1e-8)/127 and
        code = round(coeff/scale) (the FP16 cast moves a coefficient by less
        than 0.07 of a code step)."""
        dev = device or (cold_blocks[0].coeffs_K.device if cold_blocks else hot_K.device)

        def codes_of(coeffs, mm):
            absmax = torch.maximum(mm.abs().amax(-1), torch.tensor(1e-8, device=dev))
            scale = (absmax.float() / 127.0)
            codes = torch.round(coeffs.float() / scale[:, None, None]).to(torch.int8)
            return codes, scale

        if cold_blocks:
            cks, sks, bks, cvs, svs, bvs, starts = [], [], [], [], [], [], []
            for blk in cold_blocks:
                ck, sk = codes_of(blk.coeffs_K.to(dev), blk.scales_K.to(dev))
                cv, sv = codes_of(blk.coeffs_V.to(dev), blk.scales_V.to(dev))
                cks.append(ck), sks.append(sk), cvs.append(cv), svs.append(sv)
                bks.append(blk.basis_K.to(dev)), bvs.append(blk.basis_V.to(dev))
                starts.append(blk.start_position)
            stack = lambda xs: torch.stack(xs, dim=1).unsqueeze(0)   # noqa: E731
            args = (stack(cks), stack(sks), stack(bks), stack(cvs), stack(svs), stack(bvs),
                    torch.tensor([starts], device=dev))
            mmk = torch.stack([b.scales_K.to(dev).float() for b in cold_blocks], 1).unsqueeze(0)
            mmv = torch.stack([b.scales_V.to(dev).float() for b in cold_blocks], 1).unsqueeze(0)
            block_size = cold_blocks[0].block_size
        else:
            H = num_heads or hot_K.shape[1]
            D = hot_K.shape[-1]
            e8 = torch.zeros(1, H, 0, 64, 16, dtype=torch.int8, device=dev)
            args = (e8, torch.ones(1, H, 0, device=dev), torch.zeros(1, H, 0, 16, D, device=dev),
                    e8, torch.ones(1, H, 0, device=dev), torch.zeros(1, H, 0, 16, D, device=dev),
                    torch.zeros(1, 0, dtype=torch.int32, device=dev))
            mmk = mmv = None
            block_size = 512
        tail = (None, None, None)
        if hot_K is not None and hot_K.shape[2] > 0:
            hp = hot_position_ids
            if hp is None:
                start = len(cold_blocks) * block_size
                hp = torch.arange(start, start + hot_K.shape[2], device=dev)
            tail = (hot_K.to(dev, torch.float16), hot_V.to(dev, torch.float16), hp.reshape(1, -1).to(dev))
        return cls.from_tiers(*args, *tail, block_size=block_size, minmax_k=mmk, minmax_v=mmv)
