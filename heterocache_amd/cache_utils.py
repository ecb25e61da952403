"""HeteroCache: the reference's KV-cache manager on libhc kernels.

Drop-in for heterocache/cache_utils.py:610-1196 (same class and method names,
argument meaning and errors).  Storage is the tiled ragged store
(`heterocache_amd.store.KVStore`, one per layer) instead of the paged pool;
every tensor operation on the path is a libhc kernel:

  update (prefill)     keep-head copy -> hc_gather_store; full-KV tier backup
                       of satellite heads -> async D2H copy on a side stream
  update (decode)      the new token is held and appended by the fused decode
                       attention launch (or hc_append if something else
                       observes the lengths first)
  init_coefficient     hc_score + hc_select_topk + hc_set_bits (pivot sets)
  prefill_select       hc_score + hc_select_topk + hc_gather_store
  decode_attention     hc_decode_attn (replaces flash_attn_with_kvcache)
  decode_select        hc_score on the store + hc_select_topk +
                       hc_overlap_count + hc_drift_decide; the retrieval
                       gather from the host tier runs on the side stream and
                       is gated by the device trigger flag -- no host sync.

Behavioural choices (defaults; `reference_quirks=True` restores the
reference's behaviour where it differs):
  * retrieval lengths use the float32 prefill cap (the reference's float64
    lengths can exceed the prefill region by one row and overwrite the first
    generated token, heterocache/cache_utils.py:1084-1087);
  * the pivot reference set is the pivot's own (the reference indexes its
    sets by relation order but builds them in ascending pivot order,
    heterocache/cache_utils.py:1063 vs :1156-1190);
  * batch > 1 is supported per row (the reference's pool sizing and
    retrieval squeeze() assume batch 1, heterocache/cache_utils.py:704-722,
    :1093).
"""
import math
from typing import Dict, List, Optional

import numpy as np
import torch
from transformers.cache_utils import DynamicCache

from . import compress, ops
from .store import KVStore


def get_compress_len(compression_ratio, full_heads, ori_len, num_kv_heads):
    """Base budget, heterocache/cache_utils.py:15-16 (float64, truncated)."""
    return int((compression_ratio * num_kv_heads - full_heads) * ori_len / (num_kv_heads - full_heads))


class HeteroCacheConfig:
    """heterocache/cache_utils.py:41-68, plus this package's own options.

    retrieval_topk: cap on the tokens retrieved into a satellite (None =
    the reference's full budget).  window_size: observation window of the
    prefill scorer (1 = the reference's last query).  round_scores (default
    True, as the baseline compressors): the reference's casts of the scores
    to the model dtype -- logits, softmax probabilities and pooled scores
    rounded as heterocache/cache_utils.py:814-829, 1037-1057 and 1167-1187
    round them; False ranks the float32 scores (finer: fewer ties, and
    the one-pass drift check and the attention-statistics window scorer
    apply).  reference_quirks:
    float64 retrieval lengths and relation-order pivot sets, as the reference.
    chunk_tiles: decode-attention chunk (None = one resident round).
    batched_drift_check: when the model selects after attention (Llama
    order), run the drift checks of a group of layers as one launch sequence
    after the group's last layer (their results are first used by the next
    step, so the outputs are unchanged).  drift_check_groups: number of
    contiguous layer groups checked separately (1 = all layers after the
    last one; more groups start the early groups' retrieval sooner).
    overlap_drift_check: run each group's batched check and retrieval on a
    side stream, overlapping the attention of the layers outside the group;
    the group's layers wait for it before their next attention.  Off by
    default: the check and decode attention are both HBM-bound, so on their
    own they gain nothing from running together; it pays where the rest of
    the model leaves HBM bandwidth idle.
    one_pass_drift_check: let the decode attention of the leader rows report
    each step query's softmax statistics over the prompt keys
    (hc_decode_attn_stats), so that a batched check scores in one pass over
    the pivot keys (hc_score_given_stats) instead of a statistics pass that
    stores every logit and a pass over the logits.  Applies to pooling widths
    up to 9, with or without the reference's cast chain (round_scores: the
    decode launch then reports the statistics of the rounded logits);
    otherwise, and when off, the two-pass scorer runs.
    attention_stats_scoring: let the prefill attention report the softmax
    statistics of the last window_size queries (hc_prefill_attn_stats), so
    that prefill_select's observation-window scorer reads the keys once
    (hc_score_with_stats) instead of a statistics pass and a probability
    pass.  The scores are those of the same uncast float32 softmax.  It
    applies to windows of at least 32 query rows (group * window_size); with
    round_scores, for narrower windows (the default last-query scorer among
    them) or when the prefill call holds fewer than window_size queries (a
    short last chunk), the two-pass scorer runs.
    retrieval_stream: where a batched check's retrieval gathers from the
    tier arena run -- "side" (one gather per layer on a side stream, each
    layer's next attention waiting for its own rows only), "main" (one
    gather for the whole group on the check's stream) or "auto" ("side" for
    the host-pinned tier, whose reads take milliseconds over the host link;
    "main" for the HBM tier, whose gather takes tens of microseconds).
    tier_placement: where the satellites' full-KV tier lives when
    real_offload is set -- "host" (pinned host memory, retrieval read over
    the host link), "device" (an HBM arena, retrieval a device gather) or
    "auto" (device when the whole model's tier fits in tier_device_budget
    bytes, by default the device memory still free after the KV arena less
    an eighth of the device; host otherwise, and host when the device
    allocation fails).
    Without real_offload the tier is the prefill K/V itself, as in the
    reference's GPU mode.
    """

    def __init__(self, data: Optional[Dict], compression_ratio: Optional[float] = 0.5,
                 stable_threshold: Optional[float] = 0.5, real_offload: Optional[bool] = True,
                 max_gen_len: Optional[int] = 128, decode_step: Optional[int] = 4, pooling: Optional[str] = "avgpool",
                 kernel_size: Optional[int] = 5, num_attn_heads: Optional[int] = 32, num_kv_heads: Optional[int] = 8,
                 num_layers: Optional[int] = 32, retrieval_topk: Optional[int] = None, window_size: int = 1,
                 round_scores: bool = True, reference_quirks: bool = False, chunk_tiles: Optional[int] = None,
                 batched_drift_check: bool = True, drift_check_groups: int = 1, tier_placement: str = "auto",
                 tier_device_budget: Optional[int] = None, overlap_drift_check: bool = False,
                 one_pass_drift_check: bool = True, attention_stats_scoring: bool = True,
                 retrieval_stream: str = "auto"):
        self.data = data
        self.stable_threshold = stable_threshold
        self.compression_ratio = compression_ratio
        self.real_offload = real_offload
        self.max_gen_len = max_gen_len
        self.decode_step = decode_step
        self.pooling = pooling
        self.kernel_size = kernel_size
        self.quant_method = None
        self.num_attn_heads = num_attn_heads
        self.num_kv_heads = num_kv_heads
        self.num_layers = num_layers
        self.retrieval_topk = retrieval_topk
        self.window_size = window_size
        self.round_scores = round_scores
        self.reference_quirks = reference_quirks
        self.chunk_tiles = chunk_tiles
        self.batched_drift_check = batched_drift_check
        self.drift_check_groups = drift_check_groups
        if tier_placement not in ("auto", "host", "device"):
            raise ValueError(f"tier_placement must be 'auto', 'host' or 'device', not {tier_placement!r}")
        self.tier_placement = tier_placement
        self.tier_device_budget = tier_device_budget
        self.overlap_drift_check = overlap_drift_check
        self.one_pass_drift_check = one_pass_drift_check
        self.attention_stats_scoring = attention_stats_scoring
        if retrieval_stream not in ("auto", "side", "main"):
            raise ValueError(f"retrieval_stream must be 'auto', 'side' or 'main', not {retrieval_stream!r}")
        self.retrieval_stream = retrieval_stream


def _f32_caps(base, ratios, seq_len):
    """(base * ratio_f32).int() clamped to [0, L] (heterocache/cache_utils.py:793-799)."""
    r = np.asarray(ratios, dtype=np.float32)
    caps = np.trunc(np.float32(base) * r).astype(np.int64)
    return np.clip(caps, 0, seq_len)


class _DevicePack:
    """Small host arrays packed into one buffer and copied to the device in
    one transfer; add() returns a placeholder that resolve() turns into the
    device view of that array."""

    class Slot:
        __slots__ = ("off", "dtype", "n")

        def __init__(self, off, dtype, n):
            self.off, self.dtype, self.n = off, dtype, n

    _TORCH = {np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64}

    def __init__(self):
        self.parts = []
        self.words = 0   # int64 words used

    def add(self, values, dtype):
        a = np.ascontiguousarray(np.asarray(values), dtype=dtype).reshape(-1)
        slot = _DevicePack.Slot(self.words, a.dtype, a.size)
        self.parts.append((self.words, a))
        self.words += max((a.nbytes + 7) // 8, 1)
        return slot

    def upload(self, device):
        buf = np.zeros(max(self.words, 1), dtype=np.int64)
        raw = buf.view(np.uint8)
        for off, a in self.parts:
            raw[off * 8:off * 8 + a.nbytes] = a.view(np.uint8)
        return ops.to_device(buf, device, torch.int64)

    @staticmethod
    def view(dev, slot, dev32=None):
        """Device view of one added array inside the uploaded buffer (dev32:
        the same buffer viewed as int32, to slice int32 arrays in one step)."""
        if slot.dtype == np.int32:
            d32 = dev.view(torch.int32) if dev32 is None else dev32
            return d32[2 * slot.off:2 * slot.off + slot.n]
        return dev[slot.off:slot.off + slot.n]

    @staticmethod
    def resolve(obj, dev):
        """Replace every Slot inside nested dicts / tuples of obj by its view
        (one tensor slice per slot: a layer's plan holds a few dozen)."""
        dev32 = dev.view(torch.int32)
        slot_t, view = _DevicePack.Slot, _DevicePack.view

        def walk(x):
            t = type(x)
            if t is slot_t:
                return view(dev, x, dev32)
            if t is dict:
                return {k: walk(v) for k, v in x.items()}
            if t is tuple:
                return tuple([walk(v) for v in x])
            return x
        for k in list(obj):
            obj[k] = walk(obj[k])


class _LayerDrift:
    """Device state of one layer's pivot monitoring."""

    def __init__(self):
        self.leaders = []      # relation order: pivot kv-head per leader
        self.members = []      # satellite kv-heads per leader
        self.ref_bits = None   # [n_lead * B, words] int32 bitmask sets
        self.trigger = None    # [n_lead] int32
        self.qbuf = None       # [B, Hq, S, 128] buffered decode queries (view of the model-wide buffer)
        self.qlist = []        # the step queries [B, Hq, 1, 128] since the last check (references)
        self.count = 0
        self.meta = None       # device metadata and buffers, built on the first check
        self.stat_mask = 0     # steps of this cycle whose softmax statistics the decode reported


class HeteroCache(DynamicCache):
    """Compressed per-head KV cache (heterocache/cache_utils.py:610)."""

    # Workgroups of the prefill copy into the host-pinned tier.
    TIER_COPY_WORKGROUPS = 32
    # Workgroups of a retrieval gather from the host-pinned tier, and of any
    # gather beside the decode on the side stream.  Reads over the host link
    # slow concurrent HBM streaming in proportion to the reads in flight; 32
    # workgroups keep the link near its peak, and a side-stream gather of
    # one layer's rows from HBM still finishes within a layer's attention,
    # without taking the slots the decode kernel sizes its grid for.
    RETRIEVAL_WORKGROUPS = 32

    def __init__(self, cache_config):
        super().__init__()
        cfg = cache_config
        self.config = cfg
        self.num_attn_heads = cfg.num_attn_heads
        self.num_kv_heads = cfg.num_kv_heads
        self.num_layers = cfg.num_layers
        self.gqa = self.num_kv_heads != self.num_attn_heads
        self.num_key_value_groups = self.num_attn_heads // self.num_kv_heads
        self.total_kv_heads = self.num_kv_heads * self.num_layers
        self.compression_ratio = cfg.compression_ratio
        self.data = cfg.data
        self.full_heads = self.data["meta"]["counts"]["volatile"] + self.data["meta"]["counts"]["pivot"]
        self.decode_step = cfg.decode_step
        self.stable_threshold = cfg.stable_threshold
        self.device = "cpu" if cfg.real_offload else "cuda"
        self.pooling = cfg.pooling
        self.kernel_size = cfg.kernel_size
        self.quirks = bool(getattr(cfg, "reference_quirks", False))
        self.retrieval_topk = getattr(cfg, "retrieval_topk", None)
        self.window_size = int(getattr(cfg, "window_size", 1) or 1)
        self.round_scores = bool(getattr(cfg, "round_scores", True))
        self.chunk_tiles = getattr(cfg, "chunk_tiles", None)
        self.batched_check = bool(getattr(cfg, "batched_drift_check", True))
        self.overlap_check = bool(getattr(cfg, "overlap_drift_check", False))
        self.one_pass = bool(getattr(cfg, "one_pass_drift_check", True))
        self.attn_stats = bool(getattr(cfg, "attention_stats_scoring", True))
        self.attn_stats_layers = 0   # prefill layers scored with the attention's statistics
        self._side_shared = set()   # data pointers of device buffers already recorded on the side stream
        ngroups = max(1, min(int(getattr(cfg, "drift_check_groups", 1) or 1), self.num_layers))
        # Last layer of each check group (contiguous layer ranges).
        self._group_end = {((g + 1) * self.num_layers) // ngroups - 1 for g in range(ngroups)}

        self.stores = [None] * self.num_layers
        self.prefill_topk_set = [None] * self.num_layers
        self.key_cache_cpu = [None] * self.num_layers
        self.value_cache_cpu = [None] * self.num_layers
        self._tier_heads = [None] * self.num_layers   # kv-head -> head index inside the tier tensor
        self._tier_base = [0] * self.num_layers      # first tier-arena row of each layer's satellites
        self._tier = None            # (K, V) [rows, L, 128] arena of every layer's satellites, or None
        self.tier_mode = None        # "host", "device" or "prefill" (the prefill K/V kept as is)
        self._retrieval_done = [None] * self.num_layers
        self._pending = [None] * self.num_layers      # decode token awaiting its append
        self._drift = [None] * self.num_layers
        self.layer_head_capacities = [None] * self.num_layers
        self.bsz = None
        self.head_dim = None
        self.prefill_len = None
        # Chunked prefill: declared prompt length, per-layer staged K/V
        # [B, Hkv, prompt, 128], tokens staged, and the last window_size
        # query rows seen (the rows the selection scores use).
        self._prompt_len = None
        self._stage = [None] * self.num_layers
        self._staged = [0] * self.num_layers
        self._q_tail = [None] * self.num_layers
        self._seen_tokens = 0
        # The reference's multi-turn scratch caches (cleared by
        # clear_temp_kv_cache); this cache never fills them.
        self.temp_key_cache = {}
        self.temp_value_cache = {}
        self._side = None
        # Model-wide buffers: one K/V arena for every layer's rows, and the
        # drift state of every layer (per-layer objects hold views of them).
        self._arena = None
        self._tile_table = None      # int64 arena tile offsets of all rows, layer-major
        # Every layer's prefill metadata on the device, built once per cache
        # for inputs of one shape and stride: (key, [per-layer dict or None]).
        self._pplans = None
        # Per layer: (tensor key, scores, idx, counts) of init_coefficient's
        # joint selection, taken by prefill_select on the same tensors.
        self._joint_sel = [None] * self.num_layers
        self._qbuf_all = None        # [NL, B, Hq, S, 128] buffered decode queries
        # [NL, B*Hkv, G, S, 2] softmax statistics (max bound, sum) of every
        # buffered decode query over its row's prefill keys, reported by the
        # decode launches (hc_decode_attn_stats) for the one-pass check.
        self._step_stats = None
        self.one_pass_checks = 0     # batched checks scored in one pass over the pivot keys
        self._qbuf_index = {}        # layers of a batched query gather -> device index
        self._ref_bits_all = None    # [leaders * B, words] pivot reference sets
        self._trigger_all = None     # [leaders] int32 drift flags
        self._lead_base = None       # first global leader index of each layer
        self._due = []               # layers whose check waits for the batched launch
        # Whether the model calls decode_select after the step's attention
        # (Llama order: True) or before it (Qwen order: False); None until
        # the first decode_select tells.
        self._select_after_attention = None
        self._batch_meta = {}
        # Optional callable observer(event, **tensors), told about every score
        # array the cache ranks and the sets and flags it derives from them
        # (device tensors, valid on the current stream): "prefill_select"
        # (layer, rows, scores [rows, L], idx, counts), "pivot_sets" (layer,
        # pivots, scores [B * npiv, L] rows (b, pivot), K), "drift_check"
        # (row_ids [(layer, leader head, b)], scores [J, S, L], overlap [J * S],
        # trigger, trig_of, ret_idx, ret_counts).  None (the default) costs
        # nothing.
        self.observer = None

    def __del__(self):
        # The host-pinned tier is read and written by kernels through its
        # device mapping (raw pointers), which torch's pinned-memory cache
        # does not track: before the arena can return to that cache (and be
        # handed to another allocation), the side-stream work that uses it
        # must be done.
        try:
            if self._tier is not None and self._side is not None and not self._tier[0].is_cuda:
                self._side.synchronize()
        except Exception:
            pass

    # -- reference API ------------------------------------------------------
    def __bool__(self):
        return True

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self._seen_tokens if self._seen_tokens is not None else 0

    def clear_temp_kv_cache(self):
        """heterocache/cache_utils.py:1192-1196: drop the temporary caches and
        the tokens they counted.  The reference reads temp_key_cache without
        ever creating it on HeteroCache (AttributeError on a first call); here
        both start empty, so the call is a no-op until something fills them."""
        if self.temp_key_cache:
            self._seen_tokens -= next(iter(self.temp_key_cache.values())).shape[-2]
        self.temp_key_cache = {}
        self.temp_value_cache = {}

    @property
    def heads_len(self):
        """Per-layer int32 [B*Hkv] lengths (heterocache/cache_utils.py:658)."""
        for i in range(self.num_layers):
            self._flush_append(i)
        return [s.row_len if s is not None else None for s in self.stores]

    def begin_prefill(self, prompt_len):
        """Declare the prompt length ahead of a chunked prefill.

        The reference has no chunked prefill (one update per layer holds the
        whole prompt).  After this call, prefill chunks of any length (one
        token included) are staged per layer until `prompt_len` tokens have
        arrived; each chunk's attention runs over the keys staged so far, and
        the selection (init_coefficient, prefill_select), the keep-head store
        writes and the full-KV tier copy run once, on the complete prompt,
        exactly as a single-shot prefill of the same K/V would."""
        if self.bsz is not None:
            raise RuntimeError("begin_prefill must precede the first update")
        if int(prompt_len) < 1:
            raise ValueError(f"prompt length {prompt_len} must be positive")
        self._prompt_len = int(prompt_len)

    def prefill_pending(self, layer_idx):
        """True while a declared chunked prefill still expects tokens for this layer."""
        return self._prompt_len is not None and self._staged[layer_idx] < self._prompt_len

    def _stage_chunk(self, key_states, value_states, layer_idx, cache_kwargs):
        B, H, c, D = key_states.shape
        start = self._staged[layer_idx]
        end = start + c
        if end > self._prompt_len:
            raise ValueError(f"layer {layer_idx}: chunk ends at token {end}, past the declared prompt "
                             f"length {self._prompt_len}")
        if self._stage[layer_idx] is None:
            shape = (B, H, self._prompt_len, D)
            self._stage[layer_idx] = (torch.empty(shape, dtype=key_states.dtype, device=key_states.device),
                                      torch.empty(shape, dtype=value_states.dtype, device=value_states.device))
        kb, vb = self._stage[layer_idx]
        kb[:, :, start:end].copy_(key_states)
        vb[:, :, start:end].copy_(value_states)
        q = cache_kwargs.get("query_states") if cache_kwargs else None
        if q is not None:
            tail = q if self._q_tail[layer_idx] is None else torch.cat([self._q_tail[layer_idx], q], dim=2)
            self._q_tail[layer_idx] = tail[:, :, -self.window_size:]
        self._staged[layer_idx] = end
        k, v = kb[:, :, :end], vb[:, :, :end]
        if end == self._prompt_len:
            self._prefill_update(k, v, layer_idx)
            self._stage[layer_idx] = None  # the returned views keep the buffers alive
        return k, v

    def _prefill_queries(self, query_states, layer_idx):
        """Queries the selection scores read: the call's own rows, or after a
        chunked prefill the last window_size rows of the whole prompt."""
        tail = self._q_tail[layer_idx]
        if tail is None:
            return query_states
        if tail.shape[2] < self.window_size:
            raise ValueError(f"layer {layer_idx}: {tail.shape[2]} query rows staged, the observation window "
                             f"needs {self.window_size}")
        return tail

    def _side_stream(self, device):
        if self._side is None:
            self._side = torch.cuda.Stream(device=device)
        return self._side

    def drift_stream(self, device):
        """The stream the batched drift checks run on: the trigger flags and
        reference sets are ordered on it (the main stream unless checks
        overlap, overlap_drift_check)."""
        if self.overlap_check:
            return self._side_stream(device)
        return torch.cuda.current_stream(device)

    def _side_retrieval(self):
        mode = getattr(self.config, "retrieval_stream", "auto")
        if mode == "auto":
            return self.tier_mode == "host"
        return mode == "side"

    def retrieval_stream(self, device):
        """The stream the batched checks' retrieval gathers from the tier
        run on (with "side", each layer's next attention waits for its own
        rows)."""
        if self.tier_mode is not None and self._side_retrieval():
            return self._side_stream(device)
        return self.drift_stream(device)

    def _share_with_side(self, side, tensors):
        """Record device buffers allocated on the main stream as used by the
        side stream, so that their memory is not handed out again while side
        work on them is still queued."""
        for t in tensors:
            if torch.is_tensor(t) and t.is_cuda and t.data_ptr() not in self._side_shared:
                t.record_stream(side)
                self._side_shared.add(t.data_ptr())

    def _layer_row_caps(self, layer_idx):
        """Row capacities for the whole lifetime (heterocache/cache_utils.py:693-766)."""
        L, gen = self.prefill_len, self.config.max_gen_len
        keep = np.zeros(self.num_kv_heads, dtype=bool)
        keep[list(self.data["need_to_keep_counts"][layer_idx])] = True
        alloc = np.asarray(self.data["allocation_matrix"][layer_idx], dtype=np.float64)
        # float64 capacity (int() truncation, clamped to [0, L]) and float32 cap: room for both.
        c64 = np.clip(np.trunc(self.base_compress_len * alloc), 0, L).astype(np.int64)
        c32 = _f32_caps(self.base_compress_len, alloc, L)
        caps = np.where(keep, L, np.maximum(c64, c32)).astype(np.int64).tolist()
        self.layer_head_capacities[layer_idx] = caps
        return [caps[r % self.num_kv_heads] + gen for r in range(self.bsz * self.num_kv_heads)]

    def _init_storage(self, device, dtype):
        """Every layer's store in one K and one V arena, sized at the first
        prefill (all capacities follow from the prefill length)."""
        row_caps = [self._layer_row_caps(layer) for layer in range(self.num_layers)]
        tiles = [KVStore.tiles_for(c) for c in row_caps]
        n = max(sum(tiles), 1) * ops.TILE * ops.HEAD_DIM
        # Left uninitialised (clearing 17 GB at 128K took ~5 ms): every reader
        # masks by position -- decode attention past each row's length (V
        # operands zeroed), the scorers past their visible limit -- so stale
        # slots, even NaN, never reach a result.
        k = torch.empty(n, dtype=dtype, device=device)
        v = torch.empty(n, dtype=dtype, device=device)
        self._arena = (k, v)
        # Every store's row metadata in one transfer: tile offsets of all
        # rows (layer-major, which is also the model-wide tile table), then
        # per layer capacities, zero lengths, identity order, status word.
        pack = _DevicePack()
        offs, slots, base = [], [], 0
        for layer in range(self.num_layers):
            off, cap = KVStore.host_metadata(row_caps[layer], base)
            offs.append(off)
            base += tiles[layer]
            nr = len(cap)
            slots.append({"row_cap": pack.add(cap, np.int32), "row_len": pack.add(np.zeros(nr), np.int32),
                          "row_order": pack.add(np.arange(nr), np.int32), "status": pack.add([0], np.int32)})
        table = pack.add(np.concatenate(offs), np.int64)
        dev_meta = pack.upload(device)
        self._tile_table = _DevicePack.view(dev_meta, table)
        base, r0 = 0, 0
        for layer in range(self.num_layers):
            nr = len(row_caps[layer])
            meta = {k_: _DevicePack.view(dev_meta, v_) for k_, v_ in slots[layer].items()}
            meta["row_tile_off"] = self._tile_table[r0:r0 + nr]
            self.stores[layer] = KVStore(row_caps[layer], dtype, device, arena=(k, v, base), layer_idx=layer,
                                         meta=meta)
            base += tiles[layer]
            r0 += nr
        self._init_tier(device, dtype)

    def _init_tier(self, device, dtype):
        """Place the satellites' full-KV tier (see
        HeteroCacheConfig.tier_placement).  In HBM ("device", and "prefill"
        without real_offload) the tier is each layer's prefill K/V itself,
        kept by reference as the reference's GPU mode keeps it: no copy and
        no second allocation.  In host memory it is one pinned arena of
        [rows, L, 128] K and V for every layer, rows (layer, b, satellite)
        in that order."""
        if not self.config.real_offload:
            self.tier_mode = "prefill"
            return
        nsat = [len(self.data["need_to_update_counts"][layer]) for layer in range(self.num_layers)]
        rows, base = 0, []
        for n in nsat:
            base.append(rows)
            rows += self.bsz * n
        self._tier_base = base
        L = self.prefill_len
        esz = torch.empty((), dtype=dtype).element_size()
        mode = getattr(self.config, "tier_placement", "auto")
        if mode == "auto":
            # In HBM the tier keeps every layer with satellites' prefill K and V.
            kept = sum(1 for n in nsat if n) * 2 * self.bsz * self.num_kv_heads * L * self.head_dim * esz
            mode = "device" if kept <= self._tier_device_room(device) else "host"
        self.tier_mode = mode
        if rows == 0 or mode == "device":
            return
        shape = (rows, L, self.head_dim)
        self._tier = (torch.empty(shape, dtype=dtype, pin_memory=True),
                      torch.empty(shape, dtype=dtype, pin_memory=True))

    def _tier_device_room(self, device):
        """Bytes "auto" lets the full-KV tier take in HBM: tier_device_budget
        when set; otherwise the device memory still free once the KV arena
        is allocated (the driver's free memory plus what torch's allocator
        holds unused), less a reserve of an eighth of the device for the
        model's weights growth, activations and workspaces."""
        budget = getattr(self.config, "tier_device_budget", None)
        if budget is not None:
            return int(budget)
        free, total = torch.cuda.mem_get_info(device)
        cached = torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)
        return max(free + cached - total // 8, 0)

    def _layer_plan(self, layer_idx, key_states, value_states=None):
        """This layer's prefill metadata already on the device, or None when
        the inputs differ in shape or stride from those the plans were
        built for (the calls then build their metadata themselves).  The
        plans of all layers are built at the first prefill call and copied
        to the device in one transfer, so a layer's prefill launches its
        kernels without host-to-device copies of small lists."""
        if value_states is not None and (value_states.shape != key_states.shape
                                         or value_states.stride() != key_states.stride()):
            return None
        key = (tuple(key_states.shape), tuple(key_states.stride()), key_states.dtype, str(key_states.device))
        if self._pplans is None:
            self._pplans = (key,) + self._build_prefill_plans(key_states)
        if self._pplans[0] != key:
            return None
        _, plans, dev = self._pplans
        p = plans[layer_idx]
        if p is not None and not p.get("resolved"):
            _DevicePack.resolve(p, dev)   # this layer's views, made at its first use
            p["resolved"] = True
        return p

    @staticmethod
    def _tensor_key(*ts):
        """Identity of tensors' contents: storage, shape, strides and
        in-place version counter."""
        return tuple((t.data_ptr(), tuple(t.shape), tuple(t.stride()), t._version) for t in ts)

    def _build_prefill_plans(self, key_states):
        """Per layer (batch rows b, kv-heads h, row r = b * Hkv + h):
        keep-head store plan and lengths; tier copy offsets; pivot-set caps
        and the (leader, batch) row order of the reference sets; budget
        selection caps, gather plan and lengths of the compressed heads; the
        row order after the prefill.  Layers whose head data the per-call
        paths would reject get None (the per-call path raises as before)."""
        B, Hkv, L, D = self.bsz, self.num_kv_heads, self.prefill_len, self.head_dim
        s0, s1, s2 = key_states.stride()[:3]
        shape, stride = tuple(key_states.shape), tuple(key_states.stride())
        esz = key_states.element_size()
        if key_states.dim() != 4 or key_states.stride(3) != 1 or any((x * esz) % 16 for x in (s0, s1, s2)):
            return [None] * self.num_layers, None   # the per-call paths validate (and refuse) such inputs
        pack = _DevicePack()
        tier = None if self._tier is None else self._tier_arena4()[0]
        plans = []
        for layer in range(self.num_layers):
            try:
                plans.append(self._layer_prefill_plan(layer, pack, B, Hkv, L, D, s0, s1, s2, shape, stride, tier))
            except (ValueError, KeyError, IndexError):
                plans.append(None)
        return plans, pack.upload(key_states.device)

    def _layer_prefill_plan(self, layer, pack, B, Hkv, L, D, s0, s1, s2, shape, stride, tier):
        data = self.data
        p = {}
        host_len = np.zeros(B * Hkv, dtype=np.int64)
        keep = list(data["need_to_keep_counts"][layer])
        if keep:
            bh = [(b, h) for b in range(B) for h in keep]
            rows = np.asarray([b * Hkv + h for b, h in bh], dtype=np.int64)
            counts = np.full(len(rows), L, dtype=np.int64)
            p["keep"] = {"src_off": pack.add([b * s0 + h * s1 for b, h in bh], np.int64), "tok_stride": s2,
                         "src_len": L, "trig_of": None, "shape": shape, "stride": stride, "idx_off": None,
                         "counts": pack.add(counts, np.int32), "host_counts": counts,
                         "rows": pack.add(rows, np.int32), "host_rows": rows, "max_count": L}
            p["keep_len"] = (rows, counts, pack.add(rows, np.int64), p["keep"]["counts"])
            host_len[rows] = L
        sats = list(data["need_to_update_counts"][layer])
        if sats and tier is not None:
            n, r0 = len(sats), self._tier_base[layer]
            p["tier"] = {"src_off": pack.add([b * s0 + h * s1 for b in range(B) for h in sats], np.int64),
                         "dst_off": pack.add([(r0 + b * n + i) * tier.stride(1) for b in range(B) for i in range(n)],
                                             np.int64),
                         "counts": pack.add(np.full(B * n, L), np.int32), "max_count": L}
        pivots = list(data["need_to_select_counts"][layer])
        rel = data["leader_member_relations"][layer]
        K = min(self.base_compress_len, L)
        src = []
        if pivots:
            leaders = [int(h) for h in rel]
            src = ([min(i, len(pivots) - 1) for i in range(len(leaders))] if self.quirks
                   else [pivots.index(h) for h in leaders])
            p["piv_caps"] = pack.add(np.full(B * len(pivots), K), np.int32)
            p["piv_order"] = pack.add([self._score_row(b, si, len(pivots)) for si in src for b in range(B)], np.int64)
        n_c = data["need_to_compress_counts"][layer]
        if n_c and pivots and self.window_size == 1:
            # Joint scoring and selection of the compressed heads and the
            # pivots (one scorer, one selection: init_coefficient runs it,
            # prefill_select takes the compressed heads' part).  Rows
            # (b, head) over heads [0, n_c) + pivots, batch-major.
            J = n_c + len(pivots)
            caps = _f32_caps(self.base_compress_len, data["allocation_matrix"][layer][:n_c], L)
            jcaps = np.asarray([int(caps[h]) for h in range(n_c)] + [K] * len(pivots), dtype=np.int64)
            jcaps = np.tile(jcaps, B)
            jmax = int(jcaps.max())
            if jmax > 0 and caps.max() > 0:
                width = max(1, min(jmax, L))
                p["joint"] = {"heads": list(range(n_c)) + pivots, "caps": pack.add(jcaps, np.int32),
                              "max_cap": jmax, "width": width,
                              "piv_order": pack.add([b * J + n_c + si for si in src for b in range(B)], np.int64),
                              "idx_off": pack.add([(b * J + h) * width for b in range(B) for h in range(n_c)],
                                                  np.int64)}
        if n_c:
            caps = _f32_caps(self.base_compress_len, data["allocation_matrix"][layer][:n_c], L)
            rows = np.asarray([b * Hkv + h for b in range(B) for h in range(n_c)], dtype=np.int64)
            caps_rows = np.asarray([int(caps[h]) for b in range(B) for h in range(n_c)], dtype=np.int64)
            if caps_rows.max() > 0:
                W = self.window_size
                span = L - W if W > 1 else L
                width = max(1, min(int(caps_rows.max()), span + (W if W > 1 else 0)))
                cdev = pack.add(caps_rows, np.int32)
                p["caps"] = cdev
                p["max_cap"] = int(caps_rows.max())
                p["compress"] = {"src_off": pack.add([b * s0 + h * s1 for b in range(B) for h in range(n_c)], np.int64),
                                 "tok_stride": s2, "src_len": L, "trig_of": None, "shape": shape,
                                 "stride": stride, "idx_off": pack.add(np.arange(len(rows)) * width, np.int64),
                                 "counts": cdev, "host_counts": caps_rows, "rows": pack.add(rows, np.int32),
                                 "host_rows": rows, "max_count": int(caps_rows.max())}
                p["idx_width"] = width
                p["compress_len"] = (rows, caps_rows, pack.add(rows, np.int64), cdev)
                if "joint" in p:
                    p["compress_joint"] = dict(p["compress"], idx_off=p["joint"]["idx_off"])
                host_len[rows] = caps_rows
        # Row order once the prefill has set every length (longest first).
        p["order"] = pack.add(np.argsort(-host_len, kind="stable"), np.int32)
        return p

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        """heterocache/cache_utils.py:884-1005."""
        if layer_idx == 0:
            self._seen_tokens += key_states.shape[-2]
        if self.bsz is None:
            self.bsz = key_states.shape[0]
            self.head_dim = key_states.shape[-1]
            if self.head_dim != 128:
                raise ValueError(f"head_dim {self.head_dim} is not supported (128 only)")
        if not hasattr(self, "base_compress_len"):
            self.prefill_len = self._prompt_len if self._prompt_len is not None else key_states.shape[-2]
            self.base_compress_len = get_compress_len(self.compression_ratio, self.full_heads, self.prefill_len,
                                                      self.total_kv_heads)
        if self.stores[layer_idx] is None:
            self._init_storage(key_states.device, key_states.dtype)
        if self.prefill_pending(layer_idx):
            return self._stage_chunk(key_states, value_states, layer_idx, cache_kwargs)
        if key_states.shape[-2] > 1:
            self._prefill_update(key_states, value_states, layer_idx)
            return key_states, value_states
        self._flush_append(layer_idx)
        self._pending[layer_idx] = (key_states, value_states)
        return key_states, value_states

    def _prefill_update(self, key_states, value_states, layer_idx):
        """Prefill branch of update (heterocache/cache_utils.py:906-968): keep
        heads store the whole prompt; the satellites' K/V go to the tier."""
        seq_len = key_states.shape[-2]
        self.prefill_len = seq_len
        keep = self.data["need_to_keep_counts"][layer_idx]
        plan = self._layer_plan(layer_idx, key_states, value_states)
        store = self.stores[layer_idx]
        if keep and plan is not None:
            store.launch_rows(plan["keep"], key_states, value_states, set_len=False, write_len=True)
            rows, lens, drows, dlens = plan["keep_len"]
            store.set_lengths_planned(rows, lens, drows, dlens, plan["order"], on_device=True)
        elif keep:
            bh = [(b, h) for b in range(self.bsz) for h in keep]
            store.write_rows(key_states, value_states, bh, [b * self.num_kv_heads + h for b, h in bh],
                             [seq_len] * len(bh))
        self._backup_full_tier(key_states, value_states, layer_idx, plan)

    def _backup_full_tier(self, key_states, value_states, layer_idx, plan=None):
        """Full-KV tier of the satellite heads (heterocache/cache_utils.py:939-967)."""
        sats = list(self.data["need_to_update_counts"][layer_idx])
        if not sats:
            return
        if self.tier_mode in ("prefill", "device"):
            # The tier in HBM is the prefill K/V itself, kept by reference
            # (the reference's GPU mode keeps them the same way).
            self.key_cache_cpu[layer_idx] = key_states.detach()
            self.value_cache_cpu[layer_idx] = value_states.detach()
            self._tier_heads[layer_idx] = {h: h for h in sats}
            return
        L = key_states.shape[-2]
        n = len(sats)
        r0 = self._tier_base[layer_idx]
        tk, tv = self._tier_arena4()
        src = [(b, h) for b in range(self.bsz) for h in sats]
        dst = [(0, r0 + b * n + i) for b in range(self.bsz) for i in range(n)]
        tp = plan.get("tier") if plan is not None else None
        # The host-pinned arena: a few workgroups write the satellites' rows
        # straight from the prefill tensors into it at link speed, on the
        # side stream beside the compression kernels on the main stream.
        dev = key_states.device
        side = self._side_stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        if tp is not None:
            ops.copy_rows_planned(key_states, value_states, tp, tk, tv, dst_is_host=True,
                                  max_workgroups=self.TIER_COPY_WORKGROUPS, stream=side)
        else:
            ops.copy_rows(key_states, value_states, src, tk, tv, dst, [L] * len(src), dst_is_host=True,
                          max_workgroups=self.TIER_COPY_WORKGROUPS, stream=side)
        key_states.record_stream(side)
        value_states.record_stream(side)
        # The layer's rows of the arena, in the reference's [B, heads, L, 128] shape.
        self.key_cache_cpu[layer_idx] = self._tier[0][r0:r0 + self.bsz * n].view(self.bsz, n, L, self.head_dim)
        self.value_cache_cpu[layer_idx] = self._tier[1][r0:r0 + self.bsz * n].view(self.bsz, n, L, self.head_dim)
        self._tier_heads[layer_idx] = {h: i for i, h in enumerate(sats)}

    def _tier_arena4(self):
        """The tier arena as [1, rows, L, 128] K and V (gathers address its
        rows from the allocation's base)."""
        tk, tv = self._tier
        return tk.unsqueeze(0), tv.unsqueeze(0)

    def _tier_source(self, layer, b, m):
        """(K, V, (b', h')) addressing satellite m of batch row b of a layer
        in the tier: a row of the arena, or the prefill K/V in GPU mode."""
        if self.tier_mode in ("prefill", "device"):
            return self.key_cache_cpu[layer], self.value_cache_cpu[layer], (b, m)
        tk, tv = self._tier_arena4()
        n = len(self._tier_heads[layer])
        return tk, tv, (0, self._tier_base[layer] + b * n + self._tier_heads[layer][m])

    def _flush_append(self, layer_idx):
        p = self._pending[layer_idx]
        if p is None:
            return
        self._pending[layer_idx] = None
        k, v = p
        self.stores[layer_idx].append(k.reshape(-1, self.head_dim), v.reshape(-1, self.head_dim))

    def _round_dtype(self, dtype):
        return dtype if self.round_scores else None

    def prefill_stat_rows(self, query_states, layer_idx):
        """Query rows whose softmax statistics the prefill attention of this
        call should report for prefill_select's window scorer (0: none; see
        attention_stats_scoring).  The scorer reads the last window_size
        query rows over the same keys as the attention.  Windows of fewer
        than 32 query rows (group * window_size; the last-query scorers of
        prefill_select and init_coefficient among them) keep the two-pass
        scorer, which stores their few logits and is the faster form there
        (55.6 against 61.0 us for 8 heads x 128K at group 4, window 1)."""
        if not self.attn_stats or self.round_scores or self.prefill_pending(layer_idx):
            return 0
        W = self.window_size
        return W if W > 1 and self.num_key_value_groups * W >= 32 and query_states.shape[2] >= W else 0

    def init_coefficient(self, query_states, key_states, layer_idx, stats=None):
        """Pivot reference sets: top-base of the pooled last-query scores
        (heterocache/cache_utils.py:1149-1190), kept as device bitmasks.
        stats (the prefill attention's statistics, prefill_stat_rows) is
        accepted for the call's symmetry with prefill_select; the last-query
        scorer's few rows take the two-pass form, which is faster there."""
        if self.prefill_pending(layer_idx):
            return
        query_states = self._prefill_queries(query_states, layer_idx)
        pivots = list(self.data["need_to_select_counts"][layer_idx])
        rel = self.data["leader_member_relations"][layer_idx]
        st = _LayerDrift()
        self._drift[layer_idx] = st
        if not pivots:
            return
        L = key_states.shape[-2]
        G = self.num_key_value_groups
        K = min(self.base_compress_len, L)
        plan = self._layer_plan(layer_idx, key_states)
        jp = plan.get("joint") if plan is not None else None
        rd = self._round_dtype(query_states.dtype)
        if jp is not None:
            # The compressed heads are scored and selected in the same
            # launches; prefill_select takes their part if it is called with
            # these same query and key tensors.
            n_c = self.data["need_to_compress_counts"][layer_idx]
            J = len(jp["heads"])
            sc_all = compress.last_query_scores(query_states, key_states, jp["heads"], G, self.pooling,
                                                self.kernel_size, round_dtype=rd)
            idx, counts = compress.select_kept(sc_all, jp["caps"], max_cap=jp["max_cap"], round_dtype=rd)
            if idx.shape[1] != jp["width"]:
                raise RuntimeError("prefill plan: index width differs from the joint selection's")
            self._joint_sel[layer_idx] = (self._tensor_key(query_states, key_states), sc_all, idx, counts)
            scores = None
            if self.observer is not None:
                scores = sc_all.view(self.bsz, J, L)[:, n_c:].reshape(-1, L)
        else:
            scores = compress.last_query_scores(query_states, key_states, pivots, G, self.pooling, self.kernel_size,
                                                round_dtype=rd)
            if plan is not None:
                idx, _ = compress.select_kept(scores, plan["piv_caps"], max_cap=max(K, 1), round_dtype=rd)
            else:
                idx, _ = compress.select_kept(scores, [K] * scores.shape[0], max_cap=max(K, 1), round_dtype=rd)
        if self.observer is not None:
            pidx = idx if jp is None else idx.view(self.bsz, J, -1)[:, n_c:].reshape(self.bsz * len(pivots), -1)
            self.observer("pivot_sets", layer=layer_idx, pivots=pivots, scores=scores, idx=pidx, K=K)
        # Sets are stored in relation order, one row per (leader, batch).
        leaders = [int(h) for h, m in rel.items()]
        members = [list(m) for h, m in rel.items()]
        st.leaders, st.members = leaders, members
        if self.quirks:
            # The i-th relation is compared with the i-th ascending pivot's set.
            src = [min(i, len(pivots) - 1) for i in range(len(leaders))]
        else:
            src = [pivots.index(h) for h in leaders]
        # Score rows are (b, pivot position); reorder them to (leader, b).
        if jp is not None:
            order = jp["piv_order"]
        elif plan is not None:
            order = plan["piv_order"]
        else:
            order = ops.to_device([self._score_row(b, s, len(pivots)) for s in src for b in range(self.bsz)],
                                  idx.device, torch.long)
        if self._ref_bits_all is None:
            self._init_drift_buffers(idx.device, L)
        lb, B = self._lead_base[layer_idx], self.bsz
        if len(leaders) != self._lead_base[layer_idx + 1] - lb:
            raise ValueError(f"layer {layer_idx}: leader count differs from leader_member_relations")
        st.ref_bits = self._ref_bits_all[lb * B:(lb + len(leaders)) * B]
        if len(leaders):
            # Set (leader, b) takes its list from selection row order[...].
            ops.set_bits(idx, None, st.ref_bits, L, fixed_count=K, row_of=order)
            st.trigger = self._trigger_all[lb:lb + len(leaders)]
        else:
            st.trigger = torch.zeros(1, dtype=torch.int32, device=idx.device)
        self.prefill_topk_set[layer_idx] = st.ref_bits

    def _init_drift_buffers(self, device, seq_len):
        """Model-wide reference sets and trigger flags, one row per (leader,
        batch) in layer order, then relation order, then batch."""
        nlead = [len(self.data["leader_member_relations"][layer]) for layer in range(self.num_layers)]
        self._lead_base = [0]
        for n in nlead:
            self._lead_base.append(self._lead_base[-1] + n)
        total = self._lead_base[-1]
        words = max((seq_len + 31) // 32, 1)
        self._ref_bits_all = torch.zeros((total * self.bsz, words), dtype=torch.int32, device=device)
        self._trigger_all = torch.zeros(max(total, 1), dtype=torch.int32, device=device)

    @staticmethod
    def _score_row(b, pivot_pos, npiv):
        return b * npiv + pivot_pos

    def prefill_select(self, query_states, key_states, value_states, layer_idx, stats=None):
        """Compressed heads keep their top cap_h tokens in temporal order
        (heterocache/cache_utils.py:782-882).  stats: as for
        init_coefficient."""
        if self.prefill_pending(layer_idx):
            return
        query_states = self._prefill_queries(query_states, layer_idx)
        n_c = self.data["need_to_compress_counts"][layer_idx]
        if n_c == 0:
            return
        store = self.stores[layer_idx]
        L = key_states.shape[-2]
        rows = [b * self.num_kv_heads + h for b in range(self.bsz) for h in range(n_c)]
        joint = self._joint_sel[layer_idx]
        self._joint_sel[layer_idx] = None
        plan = self._layer_plan(layer_idx, key_states, value_states)
        if (joint is not None and plan is not None and "compress_joint" in plan
                and joint[0] == self._tensor_key(query_states, key_states)):
            # Selected by init_coefficient's joint launches on these tensors
            # (a plan has "compress_joint" only when some cap is above 0).
            if stats is not None:
                self.attn_stats_layers += 1
            _, sc_all, idx, counts = joint
            if self.observer is not None:
                J = len(plan["joint"]["heads"])
                self.observer("prefill_select", layer=layer_idx, rows=rows,
                              scores=sc_all.view(self.bsz, J, L)[:, :n_c].reshape(-1, L),
                              idx=idx.view(self.bsz, J, -1)[:, :n_c].reshape(self.bsz * n_c, -1),
                              counts=counts.view(self.bsz, J)[:, :n_c].reshape(-1))
            store.launch_rows(plan["compress_joint"], key_states, value_states, idx=idx, set_len=False,
                              write_len=True)
            hrows, lens, drows, dlens = plan["compress_len"]
            store.set_lengths_planned(hrows, lens, drows, dlens, plan["order"], on_device=True)
            return
        caps = _f32_caps(self.base_compress_len, self.data["allocation_matrix"][layer_idx][:n_c], L)
        caps_rows = [int(caps[h]) for b in range(self.bsz) for h in range(n_c)]
        if max(caps_rows) == 0:
            store.set_lengths([0] * len(rows), rows)
            return
        if stats is not None:
            self.attn_stats_layers += 1
        G = self.num_key_value_groups
        W = self.window_size
        rd = self._round_dtype(query_states.dtype)
        if W > 1:
            scores = compress.window_scores(query_states, key_states, range(n_c), G, W, self.pooling,
                                            self.kernel_size, window_keep=True,
                                            round_dtype=self._round_dtype(query_states.dtype), stats=stats)
        else:
            scores = compress.last_query_scores(query_states, key_states, range(n_c), G, self.pooling,
                                                self.kernel_size, round_dtype=self._round_dtype(query_states.dtype))
        if plan is not None and "compress" in plan:
            idx, counts = compress.select_kept(scores, plan["caps"], window=W if W > 1 else 0,
                                               max_cap=plan["max_cap"], round_dtype=rd)
            if idx.shape[1] != plan["idx_width"]:
                raise RuntimeError("prefill plan: index width differs from the selection's")
        else:
            plan = None
            idx, counts = compress.select_kept(scores, caps_rows, window=W if W > 1 else 0, round_dtype=rd)
        if self.observer is not None:
            self.observer("prefill_select", layer=layer_idx, rows=rows, scores=scores, idx=idx, counts=counts)
        if plan is not None:
            store.launch_rows(plan["compress"], key_states, value_states, idx=idx, set_len=False, write_len=True)
            hrows, lens, drows, dlens = plan["compress_len"]
            store.set_lengths_planned(hrows, lens, drows, dlens, plan["order"], on_device=True)
        else:
            store.write_rows(key_states, value_states, [(b, h) for b in range(self.bsz) for h in range(n_c)], rows,
                             caps_rows, idx=idx)

    def decode_attention(self, query_states, layer_idx, out=None):
        """Decode attention of q [B, Hq, 1, 128] over the layer's rows, with the
        pending token appended in the same launch.  Returns [B, 1, Hq*128]."""
        B, Hq, ql, D = query_states.shape
        if ql != 1:
            raise ValueError("decode_attention takes one query position")
        if layer_idx in self._due:
            self._flush_checks()
        store = self.stores[layer_idx]
        ev = self._retrieval_done[layer_idx]
        if ev is not None:
            torch.cuda.current_stream(query_states.device).wait_event(ev)
            self._retrieval_done[layer_idx] = None
        q = query_states.reshape(B * self.num_kv_heads, self.num_key_value_groups, D)
        p = self._pending[layer_idx]
        self._pending[layer_idx] = None
        kn = vn = None
        if p is not None:
            kn = p[0].reshape(-1, D)
            vn = p[1].reshape(-1, D)
        stat = self._step_stat_view(layer_idx, query_states)
        o = store.attend(q, 1.0 / (D ** 0.5), out=out, k_new=kn, v_new=vn, chunk_tiles=self.chunk_tiles,
                         stat_len=self.prefill_len if stat is not None else 0, stat_out=stat,
                         stat_flags=compress.ROUND_FLAGS[self._round_dtype(query_states.dtype)])
        return o.view(B, 1, Hq * D)

    def _one_pass_check(self, dtype):
        """Whether a batched drift check can score in one pass over the pivot
        keys from the decode-reported statistics (of the cast chain when the
        scores round): a pooling width hc_score_given_stats takes and fewer
        than 32 query rows per pivot."""
        return (self.one_pass and self.batched_check and self.kernel_size % 2 == 1
                and self.kernel_size <= 9 and self.num_key_value_groups * self.decode_step < 32)

    def _step_stat_view(self, layer_idx, query_states):
        """Output view [B*Hkv, G, 2] of this step's softmax statistics for a
        layer with leaders (slot: the step's position in the check cycle), or
        None.  Only the batched check of the Llama order consumes them: there
        the attention runs before the step's query is buffered, so the slot
        is the count of queries buffered so far.  In Qwen order (select
        before attention, each layer checked at once with the two-pass
        scorer) nothing is requested."""
        st = self._drift[layer_idx]
        if (st is None or not st.leaders or self._select_after_attention is False
                or not self._one_pass_check(query_states.dtype)):
            return None
        slot = st.count
        if slot >= self.decode_step:
            return None
        if self._step_stats is None:
            self._step_stats = torch.zeros((self.num_layers, self.bsz * self.num_kv_heads, self.num_key_value_groups,
                                            self.decode_step, 2), dtype=torch.float32, device=query_states.device)
        st.stat_mask |= 1 << slot
        return self._step_stats[layer_idx, :, :, slot]

    def decode_select(self, query_states, layer_idx):
        """Buffered pivot drift check and satellite retrieval
        (heterocache/cache_utils.py:1007-1147), without host syncs: after the
        first check every launch reuses device metadata built once.

        Llama order (attention already ran this step): the check is deferred
        and the checks of all layers run as one launch sequence after the
        last layer (their results are first read by the next step's
        attention).  Qwen order (select before attention): each layer checks
        at once, as its attention in this step reads the result."""
        st = self._drift[layer_idx]
        if st is None:
            st = self._drift[layer_idx] = _LayerDrift()
        if self._select_after_attention is None:
            # The attention consumed the step's pending token if it ran first.
            self._select_after_attention = self._pending[layer_idx] is None
        S = self.decode_step
        if st.qbuf is None:
            if self._qbuf_all is None:
                self._qbuf_all = torch.empty((self.num_layers, self.bsz, self.num_attn_heads, S, self.head_dim),
                                             dtype=query_states.dtype, device=query_states.device)
            st.qbuf = self._qbuf_all[layer_idx]
        # The step queries are fresh tensors the model does not touch again;
        # keeping references until the check avoids a copy per layer and step.
        if st.leaders:
            st.qlist.append(query_states)
        st.count += 1
        if st.count >= S:
            st.count = 0
            if st.leaders:
                if self.batched_check and self._pending[layer_idx] is None:
                    self._due.append(layer_idx)
                else:
                    self._gather_queries([layer_idx])
                    self._check_layer(layer_idx)
        if self._due and layer_idx in self._group_end:
            self._flush_checks()

    def _gather_queries(self, layers):
        """Buffered step queries of these layers -> qbuf [B, Hq, S, 128] each.
        With one-token queries all layers take one concatenation and one
        indexed copy into the model-wide buffer instead of one stack per
        layer (host launch time between those was idle GPU time)."""
        S = self.decode_step
        lists = []
        for layer in layers:
            st = self._drift[layer]
            lists.append(st.qlist)
            st.qlist = []
        one_token = all(len(qs) == S and qs[0].shape[2] == 1 for qs in lists)
        if self._qbuf_all is not None and one_token and len(layers) > 1:
            flat = torch.cat([q for qs in lists for q in qs], dim=2)        # [B, Hq, n*S, 128]
            B, H, _, D = flat.shape
            src = flat.view(B, H, len(layers), S, D).permute(2, 0, 1, 3, 4)  # [n, B, Hq, S, 128]
            key = tuple(layers)
            idx = self._qbuf_index.get(key)
            if idx is None:
                idx = self._qbuf_index[key] = torch.tensor(layers, dtype=torch.int64).to(flat.device)
            self._qbuf_all.index_copy_(0, idx, src)
            return
        for layer, qs in zip(layers, lists):
            torch.stack([q[:, :, -1] for q in qs], dim=2, out=self._drift[layer].qbuf)

    def _flush_checks(self):
        """Run the deferred checks: one batched launch sequence when they are
        exactly the leader layers of a contiguous layer range (the lockstep
        case), otherwise layer by layer."""
        layers, self._due = sorted(self._due), []
        self._gather_queries(layers)
        lead_layers = [l for l in range(layers[0], layers[-1] + 1)
                       if self._drift[l] is not None and self._drift[l].leaders]
        if layers == lead_layers and self._ref_bits_all is not None:
            self._check_batched(layers)
        else:
            for layer in layers:
                self._check_layer(layer)

    def _check_layer(self, layer_idx):
        """One layer's drift check and gated retrieval (two-pass scorer: any
        statistics the decode launches reported for this cycle go unused)."""
        st = self._drift[layer_idx]
        st.stat_mask = 0
        if not st.leaders or not any(st.members):
            return
        S = self.decode_step
        if st.meta is None:
            st.meta = self._drift_metadata(layer_idx, st)
        m = st.meta
        store = self.stores[layer_idx]
        L, G, B = self.prefill_len, self.num_key_value_groups, self.bsz
        K, nl = m["K"], len(st.leaders)
        # Scores of every (leader in relation order, batch row): [nl*B, S, L].
        scores = compress.pivot_step_scores(st.qbuf, store, None, None, G, L, self.pooling, self.kernel_size,
                                            round_dtype=self._round_dtype(st.qbuf.dtype),
                                            metadata=m["score_meta"], hist=m["hist"])
        # Overlaps, decision and, on trigger, the last step's top-K as the new
        # reference set -- all from the step thresholds.
        ops.drift_select(scores.view(nl * B * S, L), m["caps_K"], K, st.ref_bits, L, m["trig_of"], nl, B, S,
                         self.stable_threshold, st.trigger, m["hist"], overlap=m["overlap"])
        if m["plans"]:
            self._retrieve(layer_idx, st, scores[:, S - 1])
        if self.observer is not None:
            self.observer("drift_check", row_ids=[(layer_idx, h, b) for h in st.leaders for b in range(B)],
                          scores=scores.view(nl * B, S, L), overlap=m["overlap"], trigger=st.trigger,
                          trig_of=m["trig_of"], ret_idx=m.get("ret_idx"), ret_counts=m.get("ret_counts"))

    def _check_batched(self, layers):
        """Drift checks of a group of leader layers in one launch sequence: scores
        of every (layer, leader, batch) row read in place from the shared
        arena, one selection, overlap, decision and set update for all, one
        retrieval selection, then the gated gathers.  On the side stream
        (overlap_drift_check or a host tier) the group's layers wait for it
        at their next attention through _retrieval_done."""
        key = tuple(layers)
        bm = self._batch_meta.get(key)
        if bm is None:
            bm = self._batch_meta[key] = self._batched_metadata(layers)
        S, L, G, B = self.decode_step, self.prefill_len, self.num_key_value_groups, self.bsz
        K, J = bm["K"], bm["J"]
        qa = self._qbuf_all
        # The group's leaders are contiguous in the model-wide buffers.
        gl0, nlead = bm["lead0"], J // B
        trig = self._trigger_all[gl0:gl0 + nlead]
        bits = self._ref_bits_all[gl0 * B:(gl0 + nlead) * B]
        flags = compress.ROUND_FLAGS[self._round_dtype(qa.dtype)]
        dev = qa.device
        main = torch.cuda.current_stream(dev)
        host = self.tier_mode == "host"
        gp = bm["group_plan"]
        # The check runs on the main stream (on the side stream with
        # overlap_drift_check); the retrieval gathers of a tier arena run on
        # the side stream, one per layer, each layer's next attention waiting
        # for its own rows only.
        side = self._side_stream(dev) if self.overlap_check else main
        gather_side = self._side_stream(dev) if (gp is not None and bm["retrieve"] and self._side_retrieval()) else side
        if side is not main or gather_side is not main:
            s2 = side if side is not main else gather_side
            s2.wait_stream(main)
        if (side is not main or gather_side is not main) and not bm.get("shared"):
            # Once per check group: its buffers are the same at every check.
            bm["shared"] = True
            self._share_with_side(s2, [qa, self._arena[0], self._arena[1], self._tile_table, self._trigger_all,
                                       self._ref_bits_all]
                                  + ([] if self._tier is None else list(self._tier))
                                  + ([] if self._step_stats is None else [self._step_stats])
                                  + [t for layer, _ in bm["plans"]
                                     for t in (self.key_cache_cpu[layer], self.value_cache_cpu[layer])]
                                  + [v for v in bm.values() if torch.is_tensor(v)]
                                  + [v for v in (gp or {}).values() if torch.is_tensor(v)]
                                  + [t for layer in (gp or {}).get("layers", [])
                                     for t in (self.key_cache_cpu[layer], self.value_cache_cpu[layer])
                                     if t is not None])
        # One pass over the pivot keys when every step of the cycle had its
        # softmax statistics reported by its decode launch; otherwise the
        # statistics pass with stored logits.
        full = (1 << S) - 1
        one_pass = self._step_stats is not None and all(self._drift[layer].stat_mask == full for layer in layers)
        for layer in layers:
            self._drift[layer].stat_mask = 0
        self.one_pass_checks += int(one_pass)
        with torch.cuda.stream(side):
            if one_pass:
                scores = ops.score_given_stats(qa, bm["q_off"], qa.stride(2), qa.stride(3), self._arena[0],
                                               self._tile_table, bm["k_row"], L, G, S, self.pooling,
                                               self.kernel_size, 1.0 / math.sqrt(self.head_dim), self._step_stats,
                                               bm["st_off"], out=bm["scores"], flags=flags).view(J, S, L)
                hist = None  # the selection builds the first-digit histograms itself
            else:
                scores = ops.score(qa, bm["q_off"], qa.stride(2), qa.stride(3), self._arena[0], None, 0, L, G, S, L,
                                   self.pooling, self.kernel_size, 1.0 / math.sqrt(self.head_dim), flags=flags,
                                   row_tile_off=self._tile_table, k_row=bm["k_row"], hist=bm["hist"]).view(J, S, L)
                hist = bm["hist"]
            ops.drift_select(scores.view(J * S, L), bm["caps_K"], K, bits, L, bm["trig_of"], nlead, B, S,
                             self.stable_threshold, trig, hist, overlap=bm["overlap"])
            if bm["retrieve"]:
                ops.select_topk(scores[:, S - 1], bm["ret_caps"], L, idx=bm["ret_idx"], counts=bm["ret_counts"],
                                key_bits=compress.KEY_BITS[self._round_dtype(qa.dtype)])
            if self.observer is not None:
                self.observer("drift_check", row_ids=bm["row_ids"], scores=scores, overlap=bm["overlap"],
                              trigger=trig, trig_of=bm["trig_of"], ret_idx=bm.get("ret_idx"),
                              ret_counts=bm.get("ret_counts"))
            if bm["retrieve"] and gp is None:
                for layer, plan in bm["plans"]:
                    kc, vc = self.key_cache_cpu[layer], self.value_cache_cpu[layer]
                    self.stores[layer].launch_rows(plan, kc, vc, idx=bm["ret_idx"], src_is_host=host, stream=side,
                                                   trigger=trig, set_len=False)
        if bm["retrieve"] and gp is not None:
            # Sources: the pinned tier arena, or (in HBM) each layer's prefill
            # K/V through the plan's per-job address tables.
            tk, tv = self._tier if self._tier is not None else self._arena
            if gather_side is side:
                # Every layer of the group in one launch on the check's stream.
                ops.gather_store_groups(tk, tv, gp["src_off"], gp["group_stride"][:1], L, bm["ret_idx"],
                                        gp["idx_off"], gp["counts"], gp["dst_row"], self._arena[0], self._arena[1],
                                        self._tile_table, np.asarray([0, gp["counts"].numel()], dtype=np.int32),
                                        [gp["max_count"]], [None], src_is_host=host, trigger=trig,
                                        trig_of=gp["trig_of"], stream=side,
                                        max_workgroups=self.RETRIEVAL_WORKGROUPS if host else 0,
                                        src_k_addr=gp["k_addr"], src_v_addr=gp["v_addr"])
            else:
                # One gather per layer on the side stream (after the
                # selection), each recording its layer's event.
                gather_side.wait_stream(side)
                ops.gather_store_groups(tk, tv, gp["src_off"], gp["group_stride"], L, bm["ret_idx"], gp["idx_off"],
                                        gp["counts"], gp["dst_row"], self._arena[0], self._arena[1],
                                        self._tile_table, gp["group_begin"], gp["group_max"], gp["events"],
                                        src_is_host=host, trigger=trig, trig_of=gp["trig_of"], stream=gather_side,
                                        max_workgroups=self.RETRIEVAL_WORKGROUPS, src_k_addr=gp["k_addr"],
                                        src_v_addr=gp["v_addr"])
                for layer, ev in zip(gp["layers"], gp["events"]):
                    self._retrieval_done[layer] = ev
        if side is not main:
            # overlap_drift_check: the group's other layers wait for the whole
            # check before their next attention (its buffers are reused by
            # the next check of the main stream).
            ev = torch.cuda.Event()
            ev.record(gather_side if gather_side is not main else side)
            for layer in layers:
                if self._retrieval_done[layer] is None:
                    self._retrieval_done[layer] = ev

    def _batched_metadata(self, layers):
        """Device metadata of _check_batched; rows j follow the
        (layer, leader, batch) order of the reference sets and triggers,
        counted from the group's first leader."""
        dev = self._qbuf_all.device
        qa = self._qbuf_all
        B, Hkv, G, S, L = self.bsz, self.num_kv_heads, self.num_key_value_groups, self.decode_step, self.prefill_len
        K = min(self.base_compress_len, L)
        q_off, k_row, trig_of, ret_caps, jobs, row_ids = [], [], [], [], {}, []
        gl0 = self._lead_base[layers[0]]
        j = 0
        for layer in layers:
            st = self._drift[layer]
            lb = self._lead_base[layer] - gl0  # group-local leader index
            for i, h in enumerate(st.leaders):
                members = st.members[i]
                lens = self._retrieval_lengths(layer, members) if members else []
                mx = max(lens) if lens else 0
                for b in range(B):
                    if j != (lb + i) * B + b:
                        raise RuntimeError("batched drift rows out of the global leader order")
                    row_ids.append((layer, h, b))
                    q_off.append(layer * qa.stride(0) + b * qa.stride(1) + h * G * qa.stride(2))
                    k_row.append(layer * B * Hkv + b * Hkv + h)
                    trig_of.append(lb + i)
                    ret_caps.append(mx)
                    for mm, n in zip(members, lens):
                        if n > 0:
                            jobs.setdefault(layer, []).append((j, lb + i, b, mm, n))
                    j += 1
        J = j
        m = {"K": K, "J": J, "lead0": gl0, "row_ids": row_ids}
        m["q_off"] = torch.as_tensor(np.asarray(q_off, dtype=np.int64)).to(dev)
        m["k_row"] = torch.as_tensor(np.asarray(k_row, dtype=np.int32)).to(dev)
        # The step statistics of arena row k_row (same layer-major row order).
        m["st_off"] = torch.as_tensor(np.asarray(k_row, dtype=np.int64) * (G * S * 2)).to(dev)
        m["scores"] = torch.empty((J, S, L), dtype=torch.float32, device=dev)
        m["caps_K"] = torch.full((J * S,), K, dtype=torch.int32, device=dev)
        m["overlap"] = torch.empty(J * S, dtype=torch.int32, device=dev)
        m["hist"] = self._drift_hist(J * S, dev)
        m["trig_of"] = torch.as_tensor(np.asarray(trig_of, dtype=np.int32)).to(dev)
        m["plans"] = []
        if jobs:
            mk = max(ret_caps)
            m["ret_caps"] = torch.as_tensor(np.asarray(ret_caps, dtype=np.int32)).to(dev)
            m["ret_idx"] = torch.empty((J, max(mk, 1)), dtype=torch.int32, device=dev)
            m["ret_counts"] = torch.empty(J, dtype=torch.int32, device=dev)
            m["group_plan"] = self._group_retrieval_plan(jobs, m["ret_idx"])
            if m["group_plan"] is None:
                for layer in layers:
                    lj = jobs.get(layer)
                    if not lj:
                        continue
                    tier_heads = self._tier_heads[layer]
                    plan = self.stores[layer].plan_rows(
                        self.key_cache_cpu[layer], [(b, tier_heads[mm]) for _, _, b, mm, _ in lj],
                        [b * Hkv + mm for _, _, b, mm, _ in lj], [n for _, _, _, _, n in lj], idx=m["ret_idx"],
                        idx_rows=[jj for jj, _, _, _, _ in lj], trig_of=[t for _, t, _, _, _ in lj])
                    m["plans"].append((layer, plan))
        m.setdefault("group_plan", None)
        m["retrieve"] = bool(jobs)
        return m

    def _group_retrieval_plan(self, jobs, ret_idx):
        """One gather for every (layer, leader, batch row, satellite) retrieval
        job of a check group: sources are rows of the tier arena, destinations
        rows of the model-wide KV arena (global row = layer * B * Hkv + b *
        Hkv + satellite), each job gated by its leader's trigger flag."""
        B, Hkv, L, D = self.bsz, self.num_kv_heads, self.prefill_len, self.head_dim
        dev = ret_idx.device
        src_off, idx_off, counts, dst, trig_of, layers = [], [], [], [], [], []
        in_hbm = self._tier is None   # each layer's prefill K/V, kept by reference
        k_addr, v_addr, tok_stride = [], [], set()
        for layer, lj in sorted(jobs.items()):
            n_sat = len(self._tier_heads[layer])
            caps = self.stores[layer].host_cap
            if in_hbm:
                kc, vc = self.key_cache_cpu[layer], self.value_cache_cpu[layer]
                if kc.stride() != vc.stride():
                    return None
                tok_stride.add(kc.stride(2))
            for jj, t, b, mm, n in lj:
                if n > caps[b * Hkv + mm]:
                    raise RuntimeError(f"Layer {layer} OOM.")
                if in_hbm:
                    src_off.append(b * kc.stride(0) + mm * kc.stride(1))
                    k_addr.append(kc.data_ptr())
                    v_addr.append(vc.data_ptr())
                else:
                    src_off.append((self._tier_base[layer] + b * n_sat + self._tier_heads[layer][mm]) * L * D)
                idx_off.append(jj * ret_idx.stride(0))
                counts.append(n)
                dst.append(layer * B * Hkv + b * Hkv + mm)
                trig_of.append(t)
            layers.append(layer)
        if len(tok_stride) > 1:
            return None   # layers of different token strides: gathered layer by layer
        # One gather group per layer (jobs are in layer order), each with the
        # event its layer's next attention waits for.
        begin = [0]
        gmax = []
        for layer in layers:
            n = len(jobs[layer])
            gmax.append(max(c for *_, c in jobs[layer]))
            begin.append(begin[-1] + n)
        side = self._side_stream(dev)
        events = []
        for _ in layers:
            ev = torch.cuda.Event()
            ev.record(side)   # creates the event's handle
            events.append(ev)
        stride = tok_stride.pop() if in_hbm else D
        return {"group_begin": np.asarray(begin, dtype=np.int32), "group_max": np.asarray(gmax, dtype=np.int32),
                "group_stride": np.full(len(layers), stride, dtype=np.int64), "events": events,
                "k_addr": ops.to_device(np.asarray(k_addr, dtype=np.int64), dev) if in_hbm else None,
                "v_addr": ops.to_device(np.asarray(v_addr, dtype=np.int64), dev) if in_hbm else None,
                "src_off": ops.to_device(np.asarray(src_off, dtype=np.int64), dev),
                "idx_off": ops.to_device(np.asarray(idx_off, dtype=np.int64), dev),
                "counts": ops.to_device(np.asarray(counts, dtype=np.int32), dev),
                "dst_row": ops.to_device(np.asarray(dst, dtype=np.int32), dev),
                "trig_of": ops.to_device(np.asarray(trig_of, dtype=np.int32), dev),
                "max_count": int(max(counts)), "layers": layers}

    def _drift_metadata(self, layer_idx, st):
        """Device tensors and buffers of one layer's drift check and retrieval."""
        store = self.stores[layer_idx]
        dev = st.qbuf.device
        L, G, B, Hkv, S = self.prefill_len, self.num_key_value_groups, self.bsz, self.num_kv_heads, self.decode_step
        K = min(self.base_compress_len, L)
        nl = len(st.leaders)
        rows = [b * Hkv + h for h in st.leaders for b in range(B)]
        heads = [h for h in st.leaders for b in range(B)]
        m = {"K": K}
        m["score_meta"] = compress.pivot_step_metadata(st.qbuf, store, rows, heads, G)
        m["caps_K"] = torch.full((nl * B * S,), K, dtype=torch.int32, device=dev)
        m["overlap"] = torch.empty(nl * B * S, dtype=torch.int32, device=dev)
        m["hist"] = self._drift_hist(nl * B * S, dev)
        m["trig_of"] = torch.arange(nl, dtype=torch.int32, device=dev).repeat_interleave(B)
        # Retrieval: per leader, one gather job per (batch row, satellite).
        plans = []
        caps = [0] * (nl * B)
        for i, members in enumerate(st.members):
            if not members:
                continue
            lens = self._retrieval_lengths(layer_idx, members)
            if max(lens) == 0:
                continue
            for b in range(B):
                caps[i * B + b] = max(lens)
            plans.append((i, members, lens))
        m["plans"] = []
        if plans:
            mk = max(caps)
            m["ret_caps"] = torch.tensor(caps, dtype=torch.int32).to(dev)
            m["ret_idx"] = torch.empty((nl * B, mk), dtype=torch.int32, device=dev)
            m["ret_counts"] = torch.empty(nl * B, dtype=torch.int32, device=dev)
            # One gather for every (leader, batch row, satellite) of the layer;
            # each job is gated by its leader's trigger flag.
            jobs = [(i, b, mm, n) for i, members, lens in plans for b in range(B) for mm, n in zip(members, lens)
                    if n > 0]
            srcs = [self._tier_source(layer_idx, b, mm) for i, b, mm, n in jobs]
            m["tier"] = srcs[0][:2]
            plan = store.plan_rows(m["tier"][0], [bh for _, _, bh in srcs],
                                   [b * Hkv + mm for i, b, mm, n in jobs], [n for i, b, mm, n in jobs],
                                   idx=m["ret_idx"], idx_rows=[i * B + b for i, b, mm, n in jobs],
                                   trig_of=[i for i, b, mm, n in jobs])
            m["plans"].append(plan)
        return m

    def _drift_hist(self, rows, dev):
        """First-digit key histograms the scorer builds for the drift
        selection, one per step row; None when the group's S buffered queries
        are too many rows for the scorer to build them (the selection then
        builds its own)."""
        if self.num_key_value_groups * self.decode_step > ops.HIST_MAX_ROWS:
            return None
        return torch.empty((rows, ops.HIST_BINS), dtype=torch.int32, device=dev)

    def _retrieval_lengths(self, layer_idx, members):
        alloc = self.data["allocation_matrix"][layer_idx]
        L = self.prefill_len
        if self.quirks:
            lens = [max(min(int(self.base_compress_len * alloc[m]), L), 0) for m in members]
        else:
            lens = [int(x) for x in _f32_caps(self.base_compress_len, [alloc[m] for m in members], L)]
        if self.retrieval_topk is not None:
            lens = [min(n, int(self.retrieval_topk)) for n in lens]
        return lens

    def _retrieve(self, layer_idx, st, last_scores):
        """Gather each satellite's tokens from the full-KV tier into slots
        [0, len) of its row (heterocache/cache_utils.py:1084-1123): the
        satellite takes the ascending prefix of its leader's top-max(len)
        list of the last buffered step.  Gated by the device trigger flag;
        from the host tier it runs on the side stream, overlapping whatever
        the main stream does until this layer's next attention."""
        m = st.meta
        ops.select_topk(last_scores, m["ret_caps"], last_scores.shape[1], idx=m["ret_idx"], counts=m["ret_counts"])
        dev = last_scores.device
        main = torch.cuda.current_stream(dev)
        kc, vc = m["tier"]
        host = self.tier_mode == "host"
        store = self.stores[layer_idx]
        side = self._side_stream(dev) if host else main
        if host:
            side.wait_stream(main)
        with torch.cuda.stream(side):
            for plan in m["plans"]:
                store.launch_rows(plan, kc, vc, idx=m["ret_idx"], src_is_host=host, stream=side, trigger=st.trigger,
                                  set_len=False)
            if host:
                ev = torch.cuda.Event()
                ev.record(side)
                self._retrieval_done[layer_idx] = ev


# ---------------------------------------------------------------------------
# Baseline compressor caches (heterocache/cache_utils.py:18-41, 81-420)
# ---------------------------------------------------------------------------
class CompressionCacheConfig:
    """heterocache/cache_utils.py:18-40."""

    def __init__(self, window_size: Optional[int] = 32, compression_ratio: Optional[float] = 0.5,
                 pooling: Optional[str] = "avgpool", kernel_size: Optional[int] = 5,
                 num_attn_heads: Optional[int] = 32, num_kv_heads: Optional[int] = 8, num_layers: Optional[int] = 32):
        self.window_size = window_size
        self.compression_ratio = compression_ratio
        self.pooling = pooling
        self.kernel_size = kernel_size
        self.num_attn_heads = num_attn_heads
        self.num_kv_heads = num_kv_heads
        self.num_layers = num_layers
        self.n_init = 128


def _repeat_kv(x, n_rep):
    """K/V repeated per query head (the reference's repeat_kv): an expanded
    view materialised by one copy."""
    if n_rep == 1:
        return x
    B, H, L, D = x.shape
    return x[:, :, None].expand(B, H, n_rep, L, D).reshape(B, H * n_rep, L, D)


class BaseKVCache(DynamicCache):
    """heterocache/cache_utils.py:81-222: each layer's prompt K/V (repeated per
    query head) goes through the layer's compressor once; decode tokens are
    appended; update returns the layer's whole cache, which the model's own
    attention reads (hc_prefill_attn through the patched attention class)."""

    # Compressors of this family take K/V repeated per query head.
    repeat_kv_heads = True

    def __init__(self):
        super().__init__()
        self._seen_tokens = 0
        self.key_cache: List[torch.Tensor] = []
        self.value_cache: List[torch.Tensor] = []
        self.kv_clusters = {}
        self.kv_cluster_granularity = "layer"
        self.temp_key_cache = []
        self.temp_value_cache = []

    def __bool__(self):
        return True

    def get_kv_cluster_class_config(self, layer_idx: int, head_idx: int = None):
        raise NotImplementedError("Make sure to implement `get_kv_cluster_class_config` in a subclass.")

    def get_kv_cluster_class(self, layer_idx: int, head_idx=None):
        name, cls, config = self.get_kv_cluster_class_config(layer_idx, head_idx)
        if name not in self.kv_clusters:
            self.kv_clusters[name] = cls(**config)
        return self.kv_clusters[name]

    def compressed_kv(self, key_states, query_states, value_states, attention_mask, num_key_value_groups, layer_idx):
        if self.kv_cluster_granularity != "layer":
            raise AssertionError(f"kv_cluster_granularity {self.kv_cluster_granularity} not supported")
        cluster = self.get_kv_cluster_class(layer_idx)
        k, v = cluster.update_kv(key_states, query_states, value_states, attention_mask, num_key_value_groups)
        self.key_cache.append(k)
        self.value_cache.append(v)

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        cache_kwargs = cache_kwargs or {}
        update_global = cache_kwargs.get("update_global_past_kv", True)
        query_states = cache_kwargs["query_states"]
        groups = cache_kwargs["num_key_value_groups"]
        if self.repeat_kv_heads and key_states.size(1) != query_states.size(1):
            key_states = _repeat_kv(key_states, groups)
            value_states = _repeat_kv(value_states, groups)
        if layer_idx == 0:
            self._seen_tokens += key_states.shape[-2]
        initializing = len(self.key_cache) == layer_idx
        if initializing:
            self.compressed_kv(key_states, query_states, value_states, cache_kwargs.get("attention_mask"), groups,
                               layer_idx)
        elif update_global:
            self.key_cache[layer_idx] = torch.cat([self.key_cache[layer_idx], key_states], dim=-2)
            self.value_cache[layer_idx] = torch.cat([self.value_cache[layer_idx], value_states], dim=-2)
        elif len(self.temp_key_cache) == layer_idx:
            self.temp_key_cache.append(key_states)
            self.temp_value_cache.append(value_states)
        else:
            self.temp_key_cache[layer_idx] = torch.cat([self.temp_key_cache[layer_idx], key_states], dim=-2)
            self.temp_value_cache[layer_idx] = torch.cat([self.temp_value_cache[layer_idx], value_states], dim=-2)
        if initializing:
            return key_states, value_states
        if self.temp_key_cache:
            return (torch.cat([self.key_cache[layer_idx], self.temp_key_cache[layer_idx]], dim=-2),
                    torch.cat([self.value_cache[layer_idx], self.temp_value_cache[layer_idx]], dim=-2))
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        if len(self.key_cache) <= (layer_idx or 0):
            return 0
        return self._seen_tokens

    def to_legacy_cache(self):
        """((key, value), ...) per layer (heterocache/cache_utils.py:213-217)."""
        return tuple((self.key_cache[i], self.value_cache[i]) for i in range(len(self.key_cache)))

    @classmethod
    def from_legacy_cache(cls, past_key_values, config=None):
        """A cache holding the given per-layer (key, value) pairs
        (heterocache/cache_utils.py:219-225).  The pairs are taken as they are
        -- they are what to_legacy_cache returned, already compressed -- and
        the token count is layer 0's length.  (The reference re-enters update
        without the cache_kwargs its update requires, :142-146, so its
        version raises TypeError; replaying the pairs through update would
        compress them a second time.)  config: the subclass's constructor
        argument, for the subclasses that take one."""
        cache = cls() if config is None else cls(config)
        for k, v in past_key_values:
            cache.key_cache.append(k)
            cache.value_cache.append(v)
        cache._seen_tokens = int(past_key_values[0][0].shape[-2]) if len(past_key_values) else 0
        return cache

    def clear_temp_kv_cache(self):
        if self.temp_key_cache:
            self._seen_tokens -= self.temp_key_cache[-1].shape[-2]
        self.temp_key_cache = []
        self.temp_value_cache = []


class SnapKVCache(BaseKVCache):
    """heterocache/cache_utils.py:256-273."""

    def __init__(self, config):
        super().__init__()
        self.window_size = config.window_size
        self.compression_ratio = config.compression_ratio
        self.kernel_size = config.kernel_size
        self.pooling = config.pooling

    def get_kv_cluster_class_config(self, layer_idx: int, head_idx: int = None):
        from .kv_cluster import SnapKVCluster
        cfg = {"window_size": self.window_size, "compression_ratio": self.compression_ratio,
               "kernel_size": self.kernel_size, "pooling": self.pooling}
        return ",".join(["snapkv"] + [str(v) for v in cfg.values()]), SnapKVCluster, cfg


class PyramidKVCache(SnapKVCache):
    """heterocache/cache_utils.py:375-392."""

    def __init__(self, config):
        super().__init__(config)
        self.num_layers = config.num_layers

    def get_kv_cluster_class_config(self, layer_idx: int, head_idx: int = None):
        from .kv_cluster import PyramidKVCluster
        cfg = {"num_hidden_layers": self.num_layers, "window_size": self.window_size,
               "compression_ratio": self.compression_ratio, "kernel_size": self.kernel_size,
               "pooling": self.pooling, "layer_idx": layer_idx}
        return ",".join(["pyramidv"] + [str(v) for v in cfg.values()]), PyramidKVCluster, cfg


class H2OKVCache(BaseKVCache):
    """heterocache/cache_utils.py:237-254."""

    def __init__(self, config):
        super().__init__()
        self.window_size = config.window_size
        self.compression_ratio = config.compression_ratio
        self.kernel_size = config.kernel_size
        self.pooling = config.pooling

    def get_kv_cluster_class_config(self, layer_idx: int, head_idx: int = None):
        from .kv_cluster import H2OKVCluster
        cfg = {"window_size": self.window_size, "compression_ratio": self.compression_ratio,
               "kernel_size": self.kernel_size, "pooling": self.pooling}
        return ",".join(["h2o"] + [str(v) for v in cfg.values()]), H2OKVCluster, cfg


class StreamingLLMKVCache(SnapKVCache):
    """heterocache/cache_utils.py:395-419."""

    def get_kv_cluster_class_config(self, layer_idx: int, head_idx: int = None):
        from .kv_cluster import StreamingLLMKVCluster
        cfg = {"window_size": self.window_size, "compression_ratio": self.compression_ratio}
        return ",".join(["streamingllm"] + [str(v) for v in cfg.values()]), StreamingLLMKVCluster, cfg


class CAKECache(BaseKVCache):
    """heterocache/cache_utils.py:277-373: the prompt K/V of each layer (one
    row per KV head, not repeated) enter the cache whole, then CAKECluster
    scores the layer and evicts every layer seen so far to its budget."""

    repeat_kv_heads = False

    def __init__(self, config):
        super().__init__()
        self.window_size = config.window_size
        self.compression_ratio = config.compression_ratio
        self.kernel_size = config.kernel_size
        self.pooling = config.pooling
        self.pref_scores = []
        self.evict_scores = []
        self.layer_budget = []
        self.num_layers = config.num_layers

    def compressed_kv(self, key_states, query_states, value_states, attention_mask, num_key_value_groups, layer_idx):
        if self.kv_cluster_granularity != "layer":
            raise AssertionError(f"kv_cluster_granularity {self.kv_cluster_granularity} not supported")
        cluster = self.get_kv_cluster_class(layer_idx)
        self.key_cache.append(key_states)
        self.value_cache.append(value_states)
        cluster.update_kv(self, key_states, query_states, value_states, attention_mask, num_key_value_groups)

    def get_kv_cluster_class_config(self, layer_idx: int, head_idx: int = None):
        from .kv_cluster import CAKECluster
        cfg = {"window_size": self.window_size, "compression_ratio": self.compression_ratio,
               "kernel_size": self.kernel_size, "pooling": self.pooling}
        return ",".join(["cake"] + [str(v) for v in cfg.values()]), CAKECluster, cfg
