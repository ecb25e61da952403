"""Ragged per-head KV store of one layer (tiled head-major layout).

Replaces the reference's paged pool (`key_pools` / `value_pools` /
`block_tables` / `heads_len`, heterocache/cache_utils.py:693-766): instead of
256-token pages reached through a block table, every row (b, kv-head) owns
one contiguous run of 32-token tiles sized for its whole lifetime
(prefill budget + max_gen_len).  The reference sizes pages the same way
(cache_utils.py:719-722), so nothing is lost by dropping the indirection.
"""
import numpy as np
import torch

from . import _lib, ops

TILE = ops.TILE
HEAD_DIM = ops.HEAD_DIM


class KVStore:
    """Device buffers + row metadata of one layer's compressed cache.

    row_caps: capacity in tokens of every row (rounded up to whole tiles).
    Host mirror `host_len` tracks row_len exactly: lengths only change through
    this object's methods, so the grid of every kernel is sized without a
    device->host sync.

    arena: optional (k, v, tile_base) -- flat K and V buffers shared by
    several stores (for example every layer of a model); this store's rows
    then occupy tiles [tile_base, tile_base + total_tiles) of them and its
    row_tile_off holds arena-wide tile indices, so one launch can address
    rows of several stores through the shared base pointers.
    """

    def __init__(self, row_caps, dtype, device, arena=None, layer_idx=None, meta=None):
        caps = np.asarray(row_caps, dtype=np.int64)
        if (caps < 0).any():
            raise ValueError("negative row capacity")
        tiles = (caps + TILE - 1) // TILE
        off = np.zeros(len(caps), dtype=np.int64)
        if len(caps) > 1:
            off[1:] = np.cumsum(tiles)[:-1]
        self.rows = len(caps)
        self.layer_idx = layer_idx
        self.dtype = dtype
        self.device = torch.device(device)
        self.host_cap = tiles * TILE
        self.total_tiles = int(tiles.sum())
        if arena is None:
            n = max(self.total_tiles, 1) * TILE * HEAD_DIM
            self.k = torch.zeros(n, dtype=dtype, device=self.device)
            self.v = torch.zeros(n, dtype=dtype, device=self.device)
            self.tile_base = 0
        else:
            k, v, tile_base = arena
            if k.dtype != dtype or v.dtype != dtype or k.shape != v.shape or k.dim() != 1:
                raise ValueError("arena buffers must be flat and of the store's dtype")
            if k.device != self.device or v.device != self.device:
                raise ValueError("arena buffers must live on the store's device")
            if tile_base < 0 or (tile_base + self.total_tiles) * TILE * HEAD_DIM > k.numel():
                raise ValueError("store rows exceed the arena")
            self.k, self.v = k, v
            self.tile_base = int(tile_base)
            off = off + self.tile_base
        self.host_tile_off = off
        self.host_len = np.zeros(self.rows, dtype=np.int32)
        self._headroom = int(self.host_cap.min()) if self.rows else 0  # min over rows of cap - len
        if meta is not None:
            # Device metadata prepared by the owner of the arena (one transfer
            # for every store): views holding these rows' tile offsets
            # (int64), capacities (int32), zero lengths, the identity row
            # order and a zero status word.
            self.row_tile_off, self.row_cap = meta["row_tile_off"], meta["row_cap"]
            self.row_len, self.row_order, self.status = meta["row_len"], meta["row_order"], meta["status"]
            return
        self.row_tile_off = torch.as_tensor(off, dtype=torch.int64).to(self.device)
        self.row_cap = torch.as_tensor(self.host_cap, dtype=torch.int32).to(self.device)
        self.row_len = torch.zeros(self.rows, dtype=torch.int32, device=self.device)
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.row_order = torch.arange(self.rows, dtype=torch.int32, device=self.device)

    @staticmethod
    def host_metadata(row_caps, tile_base=0):
        """(tile offsets int64, capacities int32) of a store with these row
        capacities whose rows start at arena tile tile_base."""
        caps = np.asarray(row_caps, dtype=np.int64)
        tiles = (caps + TILE - 1) // TILE
        off = np.zeros(len(caps), dtype=np.int64)
        if len(caps) > 1:
            off[1:] = np.cumsum(tiles)[:-1]
        return off + int(tile_base), (tiles * TILE).astype(np.int32)

    @staticmethod
    def tiles_for(row_caps):
        """Tiles a store with these row capacities occupies in an arena."""
        caps = np.asarray(row_caps, dtype=np.int64)
        return int(((caps + TILE - 1) // TILE).sum())

    # -- bookkeeping -------------------------------------------------------
    def bytes_per_token(self):
        return 2 * HEAD_DIM * self.k.element_size()

    def kv_bytes(self):
        """Algorithmic K+V bytes one decode attention pass streams."""
        return int(self.host_len.sum()) * self.bytes_per_token()

    def set_lengths(self, lens, rows=None):
        rows = np.arange(self.rows) if rows is None else np.asarray(rows, dtype=np.int64)
        lens = np.asarray(lens, dtype=np.int64)
        if (lens > self.host_cap[rows]).any() or (lens < 0).any():
            raise RuntimeError("row length outside its capacity")
        self.host_len[rows] = lens
        idx = ops.to_device(rows, self.device, torch.int64)
        self.row_len.index_copy_(0, idx, ops.to_device(lens, self.device, torch.int32))
        # Longest rows are scheduled first; appends keep this order.
        order = np.argsort(-self.host_len.astype(np.int64), kind="stable").astype(np.int32)
        self._headroom = int((self.host_cap - self.host_len).min()) if self.rows else 0
        self.row_order = ops.to_device(order, self.device)

    def set_lengths_planned(self, rows, lens, dev_rows, dev_lens, dev_order=None, on_device=False):
        """set_lengths with the device copies already made: rows / lens on
        the host (numpy), dev_rows (int64) / dev_lens (int32) the same
        values on the device, dev_order (int32, optional) a row order to
        schedule by (any permutation of the rows is correct; longest first
        is the fast one), a device tensor that stays unchanged while the
        store uses it: the store schedules by it from now on, without a
        copy.  Launches one index copy and no host-to-device transfer.
        on_device: a launch already wrote the device lengths
        (launch_rows(write_len=True)); only the host mirror and the order
        are updated, and nothing is launched."""
        rows = np.asarray(rows, dtype=np.int64)
        lens = np.asarray(lens, dtype=np.int64)
        if (lens > self.host_cap[rows]).any() or (lens < 0).any():
            raise RuntimeError("row length outside its capacity")
        self.host_len[rows] = lens
        if not on_device:
            self.row_len.index_copy_(0, dev_rows, dev_lens)
        if dev_order is not None:
            if dev_order.dtype != torch.int32 or dev_order.numel() != self.rows or not dev_order.is_cuda:
                raise ValueError("dev_order must be an int32 device tensor of one entry per row")
            self.row_order = dev_order
        self._headroom = int((self.host_cap - self.host_len).min()) if self.rows else 0

    def sync_host_lengths(self, lens):
        """Set the host mirror to lengths the device already holds (after HIP
        graph replays of attend/append advanced row_len on the device); the
        device lengths and the row order are left as they are."""
        lens = np.asarray(lens, dtype=np.int64)
        if lens.shape != (self.rows,) or (lens > self.host_cap).any() or (lens < 0).any():
            raise RuntimeError("row lengths outside their capacity")
        self.host_len[:] = lens
        self._headroom = int((self.host_cap - self.host_len).min()) if self.rows else 0

    # -- writers -----------------------------------------------------------
    def plan_rows(self, src_k, src_bh, rows, counts, idx=None, idx_rows=None, trig_of=None):
        """Validate a gather and build its device metadata (see write_rows).

        The returned plan can be launched many times with launch_rows (the
        sources, index tensor and counts must keep their shapes); building
        it copies small host lists to the device, launching it does not.
        """
        rows = np.asarray(rows, dtype=np.int64)
        counts = np.asarray(counts, dtype=np.int64)
        src_bh = np.asarray(src_bh, dtype=np.int64).reshape(-1, 2)
        if len(rows) == 0:
            return None
        if len(src_bh) != len(rows) or len(counts) != len(rows):
            raise ValueError("one (b, h) source and one count per destination row")
        if (rows < 0).any() or (rows >= self.rows).any():
            raise ValueError("destination row out of range")
        if (counts > self.host_cap[rows]).any() or (counts < 0).any():
            raise RuntimeError("write exceeds a row's capacity")
        if src_k.dim() != 4 or src_k.shape[-1] != HEAD_DIM or src_k.stride(-1) != 1:
            raise ValueError("sources must be [B, H, L, 128] with unit channel stride")
        if src_k.dtype != self.dtype:
            raise TypeError("source dtype differs from the store's")
        B, H, L, _ = src_k.shape
        if (src_bh[:, 0] >= B).any() or (src_bh[:, 1] >= H).any() or (src_bh < 0).any():
            raise ValueError("source head out of range")
        if idx is None and (counts > L).any():
            raise ValueError("count exceeds the source length")
        tok_stride = src_k.stride(2)
        src_off = src_bh[:, 0] * src_k.stride(0) + src_bh[:, 1] * src_k.stride(1)
        esz = src_k.element_size()
        if (src_k.data_ptr() % 16) or (tok_stride * esz) % 16 or ((src_off * esz) % 16).any():
            raise ValueError("sources must be 16-byte aligned per token")
        dev = self.device
        idx_off = None
        if idx is not None:
            if idx.dtype != torch.int32 or idx.dim() != 2 or idx.stride(1) != 1:
                raise ValueError("idx must be int32 [n, M] with unit stride")
            r = np.arange(len(rows), dtype=np.int64) if idx_rows is None else np.asarray(idx_rows, dtype=np.int64)
            if len(r) != len(rows) or (r < 0).any() or (r >= idx.shape[0]).any():
                raise ValueError("idx_rows must name one index row per job")
            if (counts > idx.shape[1]).any():
                raise ValueError("count exceeds the index list")
            idx_off = ops.to_device(r * idx.stride(0), dev)
        if trig_of is not None:
            trig_of = ops.to_device(np.asarray(trig_of, dtype=np.int32), dev)
        return {"src_off": ops.to_device(src_off, dev), "tok_stride": tok_stride, "src_len": L,
                "trig_of": trig_of,
                "shape": tuple(src_k.shape), "stride": tuple(src_k.stride()), "idx_off": idx_off,
                "counts": ops.to_device(counts, dev, torch.int32), "host_counts": counts,
                "rows": ops.to_device(rows, dev, torch.int32), "host_rows": rows,
                "max_count": int(counts.max())}

    def launch_rows(self, plan, src_k, src_v, idx=None, src_is_host=False, stream=None, trigger=None,
                    set_len=True, max_workgroups=0, write_len=False):
        """Run a gather planned by plan_rows (no host-to-device copies).
        write_len: the gather kernel itself sets the device lengths of the
        plan's rows to their counts (the caller then updates the host mirror
        with set_lengths_planned(..., on_device=True))."""
        if plan is None:
            return
        if tuple(src_k.shape) != plan["shape"] or tuple(src_k.stride()) != plan["stride"] or \
                src_v.shape != src_k.shape or src_v.stride() != src_k.stride():
            raise ValueError("sources do not match the plan")
        if src_k.data_ptr() % 16 or src_v.data_ptr() % 16:
            raise ValueError("sources must be 16-byte aligned per token")
        if (idx is None) != (plan["idx_off"] is None):
            raise ValueError("index tensor does not match the plan")
        ops.gather_store(src_k, src_v, plan["src_off"], plan["tok_stride"], plan["src_len"], idx, plan["idx_off"],
                         plan["counts"], plan["rows"], self.k, self.v, self.row_tile_off, plan["max_count"],
                         src_is_host=src_is_host, trigger=trigger, trig_of=plan["trig_of"], stream=stream,
                         max_workgroups=max_workgroups, set_len=self.row_len if write_len else None)
        if set_len:
            self.set_lengths(plan["host_counts"], plan["host_rows"])

    def write_rows(self, src_k, src_v, src_bh, rows, counts, idx=None, idx_rows=None, src_is_host=False,
                   stream=None, trigger=None, set_len=True):
        """store[rows[j]][i] = src[b_j, h_j, idx[r_j][i]] (or token i), i < counts[j].

        src_k / src_v: [B, H, L, 128] with unit channel stride (any other
        strides), on the device or host-pinned.  src_bh: [jobs, 2] (b, h) of
        each job's source head.  idx: [n, M] int32 device tensor of source
        positions (None copies positions 0..count-1); job j reads row
        r_j = idx_rows[j] (default j).  trigger: int32 device flag gating the
        copy.
        """
        if src_k.shape != src_v.shape or src_k.stride() != src_v.stride():
            raise ValueError("K and V sources must have one shape and stride")
        plan = self.plan_rows(src_k, src_bh, rows, counts, idx=idx, idx_rows=idx_rows)
        self.launch_rows(plan, src_k, src_v, idx=idx, src_is_host=src_is_host, stream=stream, trigger=trigger,
                         set_len=set_len)

    def append(self, k_new, v_new, stream=None):
        """Write one token per row at slot len and advance every length by one.

        k_new / v_new: [rows, 128].  Raises like the reference's "OOM" when a
        row is full (heterocache/cache_utils.py:988-990).
        """
        self._check_room()
        ops.append(k_new, v_new, self.k, self.v, self.row_tile_off, self.row_len, self.row_cap, self.status,
                   stream=stream)
        self.host_len += 1
        self._headroom -= 1

    # -- readers -----------------------------------------------------------
    def read_rows(self, rows, count):
        if count > int(self.host_cap[np.asarray(rows, dtype=np.int64)].min()):
            raise ValueError("read past a row's capacity")
        return ops.store_read(self.k, self.v, self.row_tile_off, rows, count)

    def attend(self, q, scale, out=None, k_new=None, v_new=None, chunk_tiles=None,
               stream=None, num_parts=None, workspace=None, stat_len=0, stat_out=None, stat_flags=0):
        """Decode attention of q [rows, G, 128] over every row's tokens.

        With k_new / v_new [rows, 128] the decode append happens in the same
        launch: the new token is attended, stored at slot len and every
        length advances by one.  num_parts / workspace: see ops.decode_attn
        (a fixed chunk_tiles, a num_parts covering the longest lengths to
        come and an explicit workspace make the call capturable in a HIP
        graph; a replay advances the device lengths, not this object's host
        mirror).  stat_len / stat_out / stat_flags: softmax statistics of
        every row's first stat_len tokens (ops.decode_attn).
        """
        if k_new is not None:
            self._check_room()
        out = ops.decode_attn(q, self.k, self.v, self.row_tile_off, self.row_len, self.host_len, scale, out=out,
                              row_order=self.row_order, k_new=k_new, v_new=v_new, chunk_tiles=chunk_tiles,
                              stream=stream, workspace=workspace, num_parts=num_parts, row_cap=self.row_cap,
                              status=self.status, stat_len=stat_len, stat_out=stat_out, stat_flags=stat_flags)
        if k_new is not None:
            self.host_len += 1
            self._headroom -= 1
        return out

    def _oom(self):
        name = "?" if self.layer_idx is None else self.layer_idx
        return RuntimeError(f"Layer {name} OOM.")

    def _check_room(self):
        """Raise the reference's "Layer i OOM." when a row cannot take one
        more token (heterocache/cache_utils.py:988-990)."""
        if self._headroom < 1:
            raise self._oom()

    def check_status(self, stream=None):
        """After launches no host check preceded (HIP graph replays of
        attend/append): wait for the stream, clear the device status word and
        raise "Layer i OOM." if a row was at capacity.  Such a row was left
        unchanged and its output is NaN."""
        try:
            ops.read_status(self.status, clear=True, stream=stream)
        except _lib.HCError as e:
            if e.code == _lib.HC_ERR_CAPACITY:
                raise self._oom() from e
            raise
