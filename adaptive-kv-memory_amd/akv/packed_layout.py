"""Packed-layout helpers of the warm tier: measured byte accounting and the
preallocated per-head arena (akv/packed_layout.py).

``measure_packed_bytes`` follows akv/packed_layout.py:501-543: the bytes of a
quantizer dict after bit-packing -- ``codes`` as stored when the dict carries
``'bits'`` (AffineQuantizer packs them already), else packed at 2/3/4 bits --
plus the ``group_mean`` / ``group_std`` / ``scale`` / ``zero`` tensors at their
stored dtype.  Outlier channels are not counted (as in the reference).

``PackedKVArena`` is the reference's preallocated legacy-layout store
(akv/packed_layout.py:56-281) with its quantize and dequantize on the device;
``PagedKVCache`` its fp16 page pool (:283-443).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _native as nat
from . import bitpack
from ._legacy import legacy_desc, padded_dim

pack_uint4 = bitpack.pack_uint4
pack_uint3 = bitpack.pack_uint3
pack_uint2 = bitpack.pack_uint2


def measure_packed_bytes(qdata: dict, bits: int) -> int:
    """akv/packed_layout.py:501-543."""
    if "codes" not in qdata:
        return 0
    codes = qdata["codes"]
    if "bits" in qdata:
        total = codes.element_size() * codes.numel()
    else:
        total = bitpack.packed_bytes(codes, bits)
    for key in ("group_mean", "group_std", "scale", "zero"):
        t = qdata.get(key)
        if isinstance(t, torch.Tensor):
            total += t.element_size() * t.numel()
    return int(total)


@dataclass
class PackedKVConfig:
    """akv/packed_layout.py:29-55."""
    max_seq_len: int = 8192
    num_heads: int = 32
    head_dim: int = 128
    bits: int = 4          # 2, 4 or 8
    group_size: int = 128
    device: str = "cuda"
    dtype: torch.dtype = torch.float16

    @property
    def pack_factor(self) -> int:
        return 8 // self.bits

    @property
    def packed_dim(self) -> int:
        return self.head_dim // self.pack_factor

    @property
    def num_groups(self) -> int:
        return math.ceil(self.head_dim / self.group_size)


class PackedKVArena:
    """Preallocated per-head packed store (akv/packed_layout.py:56-281).

    ``data`` (H, S, D / pack_factor) uint8, ``scales`` / ``zeros`` (H, S, G) in
    ``config.dtype``: the reference's per-(head, token, group) layout.
    ``quantize_and_append`` is one ``akv_quant_pack`` launch (the ARENA layout:
    input-dtype arithmetic, clamp 1e-10, 4-bit high nibble first, 2-bit MSB
    first, 8-bit raw) whose rows are copied into the arena slots;
    ``dequantize_slice`` is one ``akv_dequant_unpack`` launch (fp32 u*s + z cast
    to ``config.dtype``).  Both are bit-exact with the reference's torch ops.
    Widths other than 2, 4 and 8 are refused at construction (the reference's
    arena fails on its first append for them)."""

    def __init__(self, config: PackedKVConfig):
        if config.bits not in (2, 4, 8):
            raise ValueError(f"PackedKVArena takes 2, 4 or 8 bits, got {config.bits}")
        if config.head_dim not in (64, 128) or config.group_size not in (32, 64, 128):
            raise NotImplementedError("the MI355X arena takes head_dim 64 or 128 and group_size 32, 64 or 128")
        self.config = config
        self._len = 0
        dev = torch.device(config.device)
        if dev.type != "cuda":
            raise RuntimeError("PackedKVArena lives on the GPU (device 'cuda')")
        H, S, Dp, G = config.num_heads, config.max_seq_len, config.packed_dim, config.num_groups
        self.data = torch.zeros(H, S, Dp, dtype=torch.uint8, device=dev)
        self.scales = torch.zeros(H, S, G, dtype=config.dtype, device=dev)
        self.zeros = torch.zeros(H, S, G, dtype=config.dtype, device=dev)
        self.positions = torch.zeros(S, dtype=torch.int32, device=dev)
        self.valid = torch.zeros(S, dtype=torch.bool, device=dev)

    @property
    def length(self) -> int:
        return self._len

    @property
    def capacity(self) -> int:
        return self.config.max_seq_len

    @property
    def bytes_used(self) -> int:
        n = self._len
        return self.data[:, :n].nbytes + self.scales[:, :n].nbytes + self.zeros[:, :n].nbytes

    def reset(self):
        self._len = 0
        self.valid[:] = False

    def quantize_and_append(self, keys: torch.Tensor) -> int:
        """akv/packed_layout.py:106-161: quantize (H, N, D) and append; when the arena
        would overflow, the N oldest tokens are evicted first.  Returns the start slot."""
        cfg = self.config
        nat.require_device(keys)
        H, N, D = keys.shape
        if H != cfg.num_heads or D != cfg.head_dim:
            raise RuntimeError(f"keys of shape {tuple(keys.shape)} do not fit an arena of {cfg.num_heads} heads "
                               f"x head_dim {cfg.head_dim}")
        if N > cfg.max_seq_len:
            raise RuntimeError(f"{N} tokens exceed the arena's {cfg.max_seq_len} slots")
        start = self._len
        if start + N > cfg.max_seq_len:
            self._evict_oldest(N)
            start = self._len
        if N == 0:
            return start
        x = keys if keys.dtype in (torch.float16, torch.bfloat16, torch.float32) else keys.float()
        x = nat.dev_contig(x)
        pD = padded_dim(D, cfg.group_size)
        G = pD // cfg.group_size
        codes = torch.empty(1, H, N, pD * cfg.bits // 8, dtype=torch.uint8, device=x.device)
        sc = torch.empty(1, H, N, G, dtype=x.dtype, device=x.device)
        ze = torch.empty_like(sc)
        lib = nat.load()
        a = nat.QuantArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.H, a.D = 1, H, D
        a.in_dtype = nat.dtype_code(x.dtype)
        a.layout = nat.QUANT_ARENA
        a.k = x.data_ptr()
        a.n_src = a.n_sel = N
        a.bits_k = a.bits_v = cfg.bits
        a.block_t = 32
        a.group_v = cfg.group_size
        a.k_codes, a.k_scale, a.k_zero = codes.data_ptr(), sc.data_ptr(), ze.data_ptr()
        nat.check(lib.akv_quant_pack(ctypes.byref(a), nat.stream_of(x)), "PackedKVArena.quantize_and_append")
        # the padding channels' codes are not kept (the reference drops them before packing)
        self.data[:, start:start + N] = codes[0, :, :, : cfg.packed_dim]
        self.scales[:, start:start + N] = sc[0].to(cfg.dtype)
        self.zeros[:, start:start + N] = ze[0].to(cfg.dtype)
        self.valid[start:start + N] = True
        self._len = start + N
        return start

    def dequantize_slice(self, start: int, end: int) -> torch.Tensor:
        """akv/packed_layout.py:163-187: (H, end - start, D) in ``config.dtype``."""
        cfg = self.config
        n = end - start
        H, D = cfg.num_heads, cfg.head_dim
        out = torch.empty(H, n, D, dtype=cfg.dtype, device=self.data.device)
        if n <= 0:
            return out
        packed = self.data[:, start:end].contiguous()
        pD = padded_dim(D, cfg.group_size)
        if pD != D:  # the kernel reads rows of the padded width; the padding codes are never used
            packed = torch.nn.functional.pad(packed, (0, (pD - D) * cfg.bits // 8))
        keep = []
        desc = legacy_desc(packed, self.scales[:, start:end], self.zeros[:, start:end], packed,
                           self.scales[:, start:end], self.zeros[:, start:end], cfg.bits, cfg.group_size, n, D,
                           warm_heads=H, sym=0, keep=keep)
        a = nat.DequantArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.Hkv, a.D = 1, H, D
        a.out_dtype = nat.dtype_code(cfg.dtype)
        a.warm = desc
        a.k_out = out.data_ptr()
        nat.check(nat.load().akv_dequant_unpack(ctypes.byref(a), nat.stream_of(out)), "PackedKVArena.dequantize_slice")
        return out

    def get_packed_slice(self, start: int, end: int):
        """akv/packed_layout.py:189-201: views of the packed codes, scales and zeros."""
        return self.data[:, start:end, :], self.scales[:, start:end, :], self.zeros[:, start:end, :]

    @staticmethod
    def _pack(data: torch.Tensor, bits: int) -> torch.Tensor:
        """akv/packed_layout.py:203-229 (torch ops on the tensor's device)."""
        if bits == 4:
            return ((data[..., 0::2] << 4) | (data[..., 1::2] & 0x0F)).to(torch.uint8)
        if bits == 2:
            return (((data[..., 0::4] & 3) << 6) | ((data[..., 1::4] & 3) << 4) | ((data[..., 2::4] & 3) << 2)
                    | (data[..., 3::4] & 3)).to(torch.uint8)
        return data

    @staticmethod
    def _unpack(packed: torch.Tensor, bits: int, target_dim: int) -> torch.Tensor:
        """akv/packed_layout.py:231-265 (float32)."""
        if bits == 4:
            u = torch.stack([(packed >> 4) & 0x0F, packed & 0x0F], dim=-1)
        elif bits == 2:
            u = torch.stack([(packed >> 6) & 3, (packed >> 4) & 3, (packed >> 2) & 3, packed & 3], dim=-1)
        else:
            return packed.float()
        return u.reshape(*packed.shape[:-1], -1).float()[..., :target_dim]

    def _evict_oldest(self, n: int):
        """akv/packed_layout.py:267-281: shift the survivors to the front."""
        if n >= self._len:
            self.reset()
            return
        remaining = self._len - n
        self.data[:, :remaining] = self.data[:, n:self._len].clone()
        self.scales[:, :remaining] = self.scales[:, n:self._len].clone()
        self.zeros[:, :remaining] = self.zeros[:, n:self._len].clone()
        self.positions[:remaining] = self.positions[n:self._len].clone()
        self.valid[:remaining] = True
        self.valid[remaining:self._len] = False
        self._len = remaining


class PagedKVCache:
    """The fp16 page pool of akv/packed_layout.py:283-443, kept on the device.

    ``k_pool`` / ``v_pool`` hold ``max_pages`` pages of (heads, page_size, head_dim)
    tokens.  Each layer's page table is a row of one int32 device tensor
    (``num_layers`` x ``max_pages``): entry j is the page of the layer's tokens
    j * page_size .. +page_size-1.  The host keeps only counts and the free list.

    ``append`` takes the pages its tokens need off the end of the free list (the
    reference's order), writes their ids into the table with one small copy, and then
    scatters all N tokens into the pool with one indexed write per pool, whatever N;
    ``get_kv`` gathers a layer's tokens with one indexed read per pool.  Freed pages are
    zeroed, all of them with one fill per pool.  ``get_page_table`` returns the layer's
    table as an int32 device tensor, as the reference does."""

    def __init__(self, num_layers: int, num_heads: int, head_dim: int, page_size: int = 16, max_pages: int = 4096,
                 dtype: torch.dtype = torch.float16, device: str = "cuda"):
        if torch.device(device).type != "cuda":
            raise RuntimeError("PagedKVCache lives on the GPU (device 'cuda')")
        self.num_layers, self.num_heads, self.head_dim = num_layers, num_heads, head_dim
        self.page_size, self.max_pages, self.dtype, self.device = page_size, max_pages, dtype, device
        self.k_pool = torch.zeros(max_pages, num_heads, page_size, head_dim, dtype=dtype, device=device)
        self.v_pool = torch.zeros_like(self.k_pool)
        self._tables = torch.zeros(num_layers, max_pages, dtype=torch.int32, device=device)
        self._free_pages = list(range(max_pages))  # taken from the end
        self._used = [False] * max_pages
        self._n_used = 0
        self._n_pages = [0] * num_layers  # pages in each layer's table
        self._seq_lens = [0] * num_layers
        self._host_tables: list[list[int]] = [[] for _ in range(num_layers)]
        self._pos = torch.arange(max_pages * page_size, dtype=torch.int64, device=device)

    # ---- page bookkeeping (host)
    def allocate_page(self) -> int:
        if not self._free_pages:
            raise RuntimeError("Page pool exhausted")
        page_id = self._free_pages.pop()
        self._used[page_id] = True
        self._n_used += 1
        return page_id

    def _release(self, page_ids) -> list:
        """Return used pages to the free list in order; the ids to clear."""
        freed = []
        for page_id in page_ids:
            if 0 <= page_id < self.max_pages and self._used[page_id]:
                self._used[page_id] = False
                self._n_used -= 1
                self._free_pages.append(page_id)
                freed.append(page_id)
        return freed

    def _clear(self, page_ids: list):
        if page_ids:
            ids = torch.tensor(page_ids, dtype=torch.int64, device=self.device)
            self.k_pool.index_fill_(0, ids, 0)
            self.v_pool.index_fill_(0, ids, 0)

    def free_page(self, page_id: int):
        self._clear(self._release([page_id]))

    # ---- data path (device)
    def _slots(self, layer_idx: int, start: int, n: int):
        """(page, offset) of the layer's tokens start .. start+n-1, as device index tensors."""
        pos = self._pos[start:start + n]
        page = self._tables[layer_idx].index_select(0, pos // self.page_size).long()
        return page, pos % self.page_size

    def append(self, layer_idx: int, keys: torch.Tensor, values: torch.Tensor):
        """keys / values (heads, N, head_dim): N tokens after the layer's last one."""
        N = int(keys.shape[1])
        if N == 0:
            return
        start = self._seq_lens[layer_idx]
        have = self._n_pages[layer_idx]
        need = -(-(start + N) // self.page_size)
        if need > have:
            new = [self.allocate_page() for _ in range(need - have)]
            self._host_tables[layer_idx].extend(new)
            self._tables[layer_idx, have:need] = torch.tensor(new, dtype=torch.int32).to(self.device, non_blocking=True)
            self._n_pages[layer_idx] = need
        page, off = self._slots(layer_idx, start, N)
        self.k_pool[page, :, off] = keys.transpose(0, 1).to(self.dtype)
        self.v_pool[page, :, off] = values.transpose(0, 1).to(self.dtype)
        self._seq_lens[layer_idx] = start + N

    def get_kv(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The layer's tokens as (heads, seq_len, head_dim) tensors."""
        n = self._seq_lens[layer_idx]
        if n == 0:
            e = torch.empty(self.num_heads, 0, self.head_dim, dtype=self.dtype, device=self.device)
            return e, e.clone()
        page, off = self._slots(layer_idx, 0, n)
        return self.k_pool[page, :, off].transpose(0, 1), self.v_pool[page, :, off].transpose(0, 1)

    def get_page_table(self, layer_idx: int) -> torch.Tensor:
        return self._tables[layer_idx, :self._n_pages[layer_idx]].clone()

    def get_seq_length(self, layer_idx: int) -> int:
        return self._seq_lens[layer_idx]

    @property
    def num_free_pages(self) -> int:
        return len(self._free_pages)

    @property
    def memory_usage_mb(self) -> float:
        return self._n_used * self.num_heads * self.page_size * self.head_dim * 2 * 2 / 1e6

    def reset(self):
        """Free every layer's pages (layer by layer, in table order) and clear them."""
        freed = []
        for layer in range(self.num_layers):
            freed += self._release(self._host_tables[layer])
            self._host_tables[layer] = []
        self._clear(freed)
        self._n_pages = [0] * self.num_layers
        self._seq_lens = [0] * self.num_layers
