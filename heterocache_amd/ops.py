"""Thin torch-tensor wrappers over the libhc C ABI.

Torch provides device memory and streams; every computation happens in the
HIP kernels of libhc.so.  Shapes, dtypes and devices are checked here, on the
host, before any kernel is launched.
"""
import ctypes

import numpy as np
import torch

from . import _lib

HEAD_DIM = 128
TILE = 32

_DTYPES = {torch.float32: _lib.HC_DTYPE_F32, torch.float16: _lib.HC_DTYPE_F16, torch.bfloat16: _lib.HC_DTYPE_BF16}


def dtype_code(dt):
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


def to_device(values, device, dtype=None):
    """Small host metadata (a list or numpy array) as a device tensor without
    a host sync: staged in pinned memory (torch's caching host allocator)
    and copied asynchronously on the current stream.  A plain .to(device)
    of pageable memory synchronises the stream, draining the GPU at every
    metadata copy."""
    t = torch.as_tensor(np.asarray(values), dtype=dtype)
    if t.device.type != "cpu":
        return t.to(device)
    return t.pin_memory().to(device, non_blocking=True)


def _ptr(t):
    # ctypes passes a Python int (or None) for a c_void_p argument as is.
    return t.data_ptr() if t is not None else None


def _stream(stream, like):
    """Raw HIP stream: the given one, else the current stream of the device
    of tensor `like` (read without constructing a torch Stream object)."""
    if stream is not None:
        return stream.cuda_stream
    return torch._C._cuda_getCurrentRawStream(like.device.index)


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("libhc ops need tensors on a ROCm device")


class Workspace:
    """Grow-only, zero-initialised per-device scratch buffer.

    hc_select_topk's histograms must start at zero (each call leaves them
    zeroed again), so the buffer is zero-filled when (re)allocated; the
    decode workspace needs no initialisation.  Launches on one stream reuse
    it; work on another stream needs its own instance.
    """

    def __init__(self):
        self._buf = {}

    def get(self, device, nbytes):
        dev = torch.device(device)
        key = dev.index if dev.index is not None else torch.cuda.current_device()
        buf = self._buf.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                torch.cuda.current_stream(dev).synchronize()
            buf = torch.zeros(max(nbytes, 1 << 22), dtype=torch.uint8, device=dev)
            self._buf[key] = buf
        return buf


WORKSPACE = Workspace()
# hc_select_topk keeps self-clearing histograms in this buffer.
SELECT_HIST = Workspace()
# Bins of the first-digit key histogram hc_score builds for hc_drift_select,
# and the query rows below which it can (the logit-store path).
HIST_BINS = 4096
HIST_MAX_ROWS = 31


def _lens_i32(host_row_len):
    lens = np.asarray(host_row_len)
    if lens.dtype != np.int32 or not lens.flags.c_contiguous:
        lens = np.ascontiguousarray(lens, dtype=np.int32)
    return lens


def decode_num_parts(host_row_len, chunk_tiles):
    """Workgroups of one decode launch: chunks of chunk_tiles 32-token tiles
    per row (an empty row still takes one)."""
    lens = _lens_i32(host_row_len)
    n = _lib.load().hc_decode_num_parts(lens.ctypes.data, len(lens), int(chunk_tiles))
    if n < 0:
        raise ValueError("bad arguments to hc_decode_num_parts")
    return n


def decode_chunk_tiles(host_row_len, group, dtype):
    """The chunk size whose grid fills the current device in one resident
    round for these lengths (hc_decode_chunk_tiles)."""
    lens = _lens_i32(host_row_len)
    n = _lib.load().hc_decode_chunk_tiles(dtype_code(dtype), lens.ctypes.data, len(lens), int(group))
    _lib.check(min(n, 0))
    return n


def decode_attn(q, kstore, vstore, row_tile_off, row_len, host_row_len, scale, out=None, row_order=None,
                k_new=None, v_new=None, chunk_tiles=None, stream=None, workspace=None, num_parts=None,
                row_cap=None, status=None, stat_len=0, stat_out=None, stat_flags=0):
    """out[r, g] = softmax(scale * q[r, g] . K_r^T) V_r over row_len[r] tokens.

    q: [rows, G, 128]; host_row_len: host copy of the lengths (sizes the grid).
    With k_new/v_new [rows, 128] the new token is appended and attended in the
    same launch; row_len advances by one (the caller advances its mirror).
    row_cap (int32 [rows], required with k_new): a row at capacity is left
    unchanged, its output is NaN and bit 0 of status (int32 device word,
    optional) is set -- read it with read_status.
    chunk_tiles: tiles per workgroup; None picks the one-round chunk for
    these lengths.  num_parts: grid size, at least what these lengths need;
    a larger grid (surplus workgroups exit at once) lets a captured HIP graph
    replay while the device lengths grow.  workspace: a uint8 device tensor
    of at least hc_decode_workspace_size bytes (default: a shared buffer).
    stat_len > 0 with stat_out (float32 [rows, G, 2] view, any strides with
    a unit last-dim stride): each row's softmax statistics (base-2 max bound,
    sum of exp2 against it) over its first stat_len tokens
    (hc_decode_attn_stats); stat_flags HC_SCORE_ROUND_BF16 / _F16: of the
    reference's cast chain of the logits instead.
    """
    lib = _lib.load()
    _require_cuda(q, kstore, vstore, row_tile_off, row_len, row_order, k_new, v_new)
    if q.dim() != 3 or q.shape[-1] != HEAD_DIM:
        raise ValueError(f"q must be [rows, G, {HEAD_DIM}], got {tuple(q.shape)}")
    rows, G, _ = q.shape
    if row_len.numel() != rows or row_tile_off.numel() != rows or len(host_row_len) != rows:
        raise ValueError("row metadata does not match q's row count")
    if row_len.dtype != torch.int32 or row_tile_off.dtype != torch.int64:
        raise TypeError("row_len must be int32 and row_tile_off int64")
    if kstore.dtype != q.dtype or vstore.dtype != q.dtype:
        raise TypeError("q and the store must share a dtype")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new go together")
    _require_cuda(row_cap, status)
    if k_new is not None:
        if row_cap is None or row_cap.dtype != torch.int32 or row_cap.numel() != rows:
            raise ValueError("a fused append needs row_cap, int32 [rows]")
        if status is not None and (status.dtype != torch.int32 or status.numel() < 1):
            raise ValueError("status must be an int32 device word")
        if k_new.shape != (rows, HEAD_DIM) or v_new.shape != (rows, HEAD_DIM):
            raise ValueError(f"k_new/v_new must be [{rows}, {HEAD_DIM}]")
        if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
            raise TypeError("k_new/v_new must share q's dtype")
        k_new = k_new.contiguous()
        v_new = v_new.contiguous()
        host_row_len = _lens_i32(host_row_len) + np.int32(1)
    if row_order is not None and (row_order.dtype != torch.int32 or row_order.numel() != rows):
        raise ValueError("row_order must be an int32 permutation of the rows")
    q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous() or out.device != q.device:
        raise ValueError("out must be a contiguous tensor of q's shape, dtype and device")
    if chunk_tiles is None:
        chunk_tiles = decode_chunk_tiles(host_row_len, G, q.dtype)
    nparts = decode_num_parts(host_row_len, chunk_tiles)
    if num_parts is not None:
        if int(num_parts) < nparts:
            raise ValueError(f"num_parts {num_parts} is below the {nparts} parts these lengths need")
        nparts = int(num_parts)
    nbytes = lib.hc_decode_workspace_size(rows, G, nparts)
    ws = workspace if workspace is not None else WORKSPACE.get(q.device, nbytes)
    st_ptr = _ptr(status) if k_new is not None else None
    if stat_len:
        _require_cuda(stat_out)
        if (stat_out is None or stat_out.dtype != torch.float32 or tuple(stat_out.shape) != (rows, G, 2)
                or stat_out.stride(2) != 1 or stat_out.device != q.device):
            raise ValueError(f"stat_out must be a float32 [{rows}, {G}, 2] device view with unit last stride")
        _lib.check(lib.hc_decode_attn_stats(
            dtype_code(q.dtype), _ptr(q), _ptr(kstore), _ptr(vstore), _ptr(row_tile_off), _ptr(row_len),
            _ptr(row_cap), _ptr(row_order), rows, G, float(scale), _ptr(k_new), _ptr(v_new), _ptr(out), _ptr(ws),
            ws.numel(), nparts, int(chunk_tiles), st_ptr, int(stat_len), _ptr(stat_out), stat_out.stride(0),
            stat_out.stride(1), int(stat_flags), _stream(stream, q)))
        return out
    _lib.check(lib.hc_decode_attn(dtype_code(q.dtype), _ptr(q), _ptr(kstore), _ptr(vstore), _ptr(row_tile_off),
                                  _ptr(row_len), _ptr(row_cap), _ptr(row_order), rows, G, float(scale), _ptr(k_new),
                                  _ptr(v_new), _ptr(out), _ptr(ws), ws.numel(), nparts, int(chunk_tiles),
                                  st_ptr, _stream(stream, q)))
    return out


def stream_read(buf, workgroups_per_cu=8, sink=None, stream=None):
    """Read a device buffer once with nontemporal 16-byte loads and discard
    it (hc_stream_read): timed over a buffer larger than the last-level
    cache, the device's streaming-read ceiling."""
    lib = _lib.load()
    _require_cuda(buf)
    if not buf.is_contiguous():
        raise ValueError("buf must be contiguous")
    if sink is None:
        sink = torch.zeros(1, dtype=torch.float32, device=buf.device)
    _lib.check(lib.hc_stream_read(_ptr(buf), buf.numel() * buf.element_size(), _ptr(sink), int(workgroups_per_cu),
                                  _stream(stream, buf)))
    return sink


def read_status(status, clear=True, stream=None):
    """Wait for the stream and read the device status word of hc_append /
    hc_decode_attn (zeroing it when clear).  Returns the word; raises
    HCError(HC_ERR_CAPACITY) when a row was at capacity."""
    _require_cuda(status)
    if status.dtype != torch.int32 or status.numel() < 1:
        raise ValueError("status must be an int32 device word")
    val = ctypes.c_int32(0)
    _lib.check(_lib.load().hc_read_status(_ptr(status), int(bool(clear)), ctypes.addressof(val),
                                          _stream(stream, status)))
    return val.value


def gather_store(src_k, src_v, src_off, src_tok_stride, src_len, idx, idx_off, count, dst_row, kstore, vstore, row_tile_off,
                 max_count, src_is_host=False, trigger=None, trig_of=None, stream=None, max_workgroups=0, set_len=None):
    """store[dst_row[j]][i] = src[src_off[j] + idx[idx_off[j] + i] * stride], i < count[j].

    max_workgroups: grid cap (0: the library default for the source kind).
    set_len: the store's int32 row lengths; row dst_row[j]'s becomes count[j]."""
    lib = _lib.load()
    _require_cuda(src_off, count, dst_row, kstore, vstore, row_tile_off, idx, idx_off, trigger, trig_of, set_len)
    if src_is_host:
        if src_k.is_cuda or not src_k.is_pinned() or not src_v.is_pinned():
            raise ValueError("host sources must be pinned CPU tensors")
    else:
        _require_cuda(src_k, src_v)
    if src_k.dtype != kstore.dtype or src_v.dtype != vstore.dtype:
        raise TypeError("source and store dtypes differ")
    for name, t, dt in (("src_off", src_off, torch.int64), ("count", count, torch.int32),
                        ("dst_row", dst_row, torch.int32), ("idx", idx, torch.int32),
                        ("idx_off", idx_off, torch.int64), ("trigger", trigger, torch.int32),
                        ("trig_of", trig_of, torch.int32), ("set_len", set_len, torch.int32)):
        if t is not None and t.dtype != dt:
            raise TypeError(f"{name} must be {dt}")
    njobs = count.numel()
    _lib.check(lib.hc_gather_store(dtype_code(kstore.dtype), _ptr(src_k), _ptr(src_v), int(bool(src_is_host)),
                                   _ptr(src_off), int(src_tok_stride), int(src_len), _ptr(idx), _ptr(idx_off), _ptr(count),
                                   _ptr(dst_row), _ptr(kstore), _ptr(vstore), _ptr(row_tile_off), njobs,
                                   int(max_count), _ptr(trigger), _ptr(trig_of), int(max_workgroups), _ptr(set_len),
                                   _stream(stream, kstore)))


def gather_store_groups(src_k, src_v, src_off, group_tok_stride, src_len, idx, idx_off, count, dst_row, kstore,
                        vstore, row_tile_off, group_begin, group_max_count, events, src_is_host=False, trigger=None,
                        trig_of=None, stream=None, max_workgroups=0, src_k_addr=None, src_v_addr=None):
    """gather_store over consecutive job groups, one launch per group, each
    followed by a record of that group's event (hc_gather_store_groups).

    group_begin (int32, ngroups + 1), group_max_count (int32, ngroups) and
    group_tok_stride (int64, ngroups): host numpy arrays.  events: one
    torch.cuda.Event (or None) per group; each is recorded on `stream` once
    its group's rows are written.  src_k_addr / src_v_addr: optional int64
    device tensors of one source address per job (src_off is added to it);
    src_k / src_v then only give the dtype."""
    lib = _lib.load()
    _require_cuda(src_off, count, dst_row, kstore, vstore, row_tile_off, idx, idx_off, trigger, trig_of, src_k_addr,
                  src_v_addr)
    if src_k_addr is not None:
        if src_v_addr is None or src_k_addr.dtype != torch.int64 or src_k_addr.numel() != count.numel() or \
                src_v_addr.dtype != torch.int64 or src_v_addr.numel() != count.numel():
            raise ValueError("src_k_addr and src_v_addr must be int64 tensors of one address per job")
        if src_is_host:
            raise ValueError("per-job source addresses are device addresses")
    if src_is_host:
        if src_k.is_cuda or not src_k.is_pinned() or not src_v.is_pinned():
            raise ValueError("host sources must be pinned CPU tensors")
    else:
        _require_cuda(src_k, src_v)
    if src_k.dtype != kstore.dtype or src_v.dtype != vstore.dtype:
        raise TypeError("source and store dtypes differ")
    gb = np.ascontiguousarray(group_begin, dtype=np.int32)
    gm = np.ascontiguousarray(group_max_count, dtype=np.int32)
    gs = np.ascontiguousarray(group_tok_stride, dtype=np.int64)
    ng = len(gm)
    if len(gb) != ng + 1 or len(gs) != ng or len(events) != ng:
        raise ValueError("group arrays and events must describe the same groups")
    if gb[-1] != count.numel():
        raise ValueError(f"groups cover {gb[-1]} jobs, count holds {count.numel()}")
    handles = (ctypes.c_void_p * max(ng, 1))(*[(e.cuda_event if e is not None else 0) for e in events])
    _lib.check(lib.hc_gather_store_groups(dtype_code(kstore.dtype), _ptr(src_k), _ptr(src_v), int(bool(src_is_host)),
                                          _ptr(src_off), gs.ctypes.data, int(src_len), _ptr(idx), _ptr(idx_off),
                                          _ptr(count), _ptr(dst_row), _ptr(kstore), _ptr(vstore), _ptr(row_tile_off),
                                          ng, gb.ctypes.data, gm.ctypes.data, _ptr(trigger), _ptr(trig_of),
                                          int(max_workgroups), handles, _ptr(src_k_addr), _ptr(src_v_addr),
                                          _stream(stream, kstore)))


def copy_rows(src_k, src_v, src_bh, dst_k, dst_v, dst_bh, counts, dst_is_host=False, max_workgroups=32,
              stream=None):
    """dst[b', h', t] = src[b, h, t] for t < counts[j], (b, h) = src_bh[j], (b', h') = dst_bh[j].

    src / dst: [B, H, L, 128] tensors with unit channel stride; dst may be a
    pinned CPU tensor (dst_is_host).  At most max_workgroups workgroups run
    the copy.  With `stream`, that stream first waits for the current one
    (which builds the small offset tensors).
    """
    lib = _lib.load()
    _require_cuda(src_k, src_v)
    if dst_is_host:
        if dst_k.is_cuda or not dst_k.is_pinned() or not dst_v.is_pinned():
            raise ValueError("host destinations must be pinned CPU tensors")
    else:
        _require_cuda(dst_k, dst_v)
    for t in (src_k, src_v, dst_k, dst_v):
        if t.dim() != 4 or t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
            raise ValueError("sources and destinations must be [B, H, L, 128] with unit channel stride")
    if src_k.stride() != src_v.stride() or dst_k.stride() != dst_v.stride():
        raise ValueError("K and V must share strides")
    if not (src_k.dtype == src_v.dtype == dst_k.dtype == dst_v.dtype):
        raise TypeError("sources and destinations must share a dtype")
    src_bh = np.asarray(src_bh, dtype=np.int64).reshape(-1, 2)
    dst_bh = np.asarray(dst_bh, dtype=np.int64).reshape(-1, 2)
    counts = np.asarray(counts, dtype=np.int64)
    if not (len(src_bh) == len(dst_bh) == len(counts)):
        raise ValueError("one source head, destination head and count per job")
    if len(counts) == 0:
        return
    for bh, t in ((src_bh, src_k), (dst_bh, dst_k)):
        if (bh < 0).any() or (bh[:, 0] >= t.shape[0]).any() or (bh[:, 1] >= t.shape[1]).any():
            raise ValueError("head index out of range")
    if (counts < 0).any() or (counts > src_k.shape[2]).any() or (counts > dst_k.shape[2]).any():
        raise ValueError("count exceeds a source or destination length")
    dev = src_k.device
    plan = {"src_off": to_device(src_bh[:, 0] * src_k.stride(0) + src_bh[:, 1] * src_k.stride(1), dev, torch.int64),
            "dst_off": to_device(dst_bh[:, 0] * dst_k.stride(0) + dst_bh[:, 1] * dst_k.stride(1), dev, torch.int64),
            "counts": to_device(counts, dev, torch.int32), "max_count": int(counts.max())}
    copy_rows_planned(src_k, src_v, plan, dst_k, dst_v, dst_is_host, max_workgroups, stream)


def copy_rows_planned(src_k, src_v, plan, dst_k, dst_v, dst_is_host=False, max_workgroups=32, stream=None):
    """copy_rows with its device metadata already built: plan holds int64
    device tensors src_off / dst_off (element offsets of each job's head),
    int32 counts and the host max_count (the caller validated them against
    these tensors' shapes).  With `stream`, that stream first waits for the
    current one."""
    lib = _lib.load()
    if stream is not None:
        # The launch stream waits for the metadata (and whatever produced the
        # sources) on the current stream.
        stream.wait_stream(torch.cuda.current_stream(src_k.device))
        for t in (plan["src_off"], plan["dst_off"], plan["counts"]):
            t.record_stream(stream)
    _lib.check(lib.hc_copy_rows(dtype_code(src_k.dtype), _ptr(src_k), _ptr(src_v), _ptr(plan["src_off"]),
                                src_k.stride(2), _ptr(dst_k), _ptr(dst_v), int(bool(dst_is_host)),
                                _ptr(plan["dst_off"]), dst_k.stride(2), _ptr(plan["counts"]),
                                plan["counts"].numel(), int(plan["max_count"]), int(max_workgroups),
                                _stream(stream, src_k)))


def prefill_attn(q, k, v, scale, out=None, stream=None, stat_out=None):
    """Causal attention of the last Lq positions over Lk keys (hc_prefill_attn).

    q: [B, Hq, Lq, 128]; k, v: [B, Hkv, Lk, 128] (any batch/head/token
    strides, unit channel stride; Lq <= Lk, query i sits at position
    Lk - Lq + i).  Returns out [B, Lq, Hq, 128] (or writes the given `out`,
    which may be any view of that shape with unit channel stride).
    stat_out: optional contiguous float32 [B, Hq, W, 2] (W <= Lq) that
    receives the softmax statistics (M, L) of the last W queries of each
    head (hc_prefill_attn_stats), the normalisers the window scorers reuse.
    """
    lib = _lib.load()
    _require_cuda(q, k, v, out)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k and v must be [B, H, L, 128]")
    B, Hq, Lq, D = q.shape
    if D != HEAD_DIM or k.shape[-1] != HEAD_DIM or v.shape != k.shape or k.shape[0] != B:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}: head_dim must be 128 "
                         "and k, v must share [B, Hkv, Lk]")
    Hkv, Lk = k.shape[1], k.shape[2]
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads are not a multiple of {Hkv} KV heads")
    if Lq > Lk:
        raise ValueError(f"{Lq} queries exceed {Lk} keys")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k and v must share a dtype")
    if out is None:
        out = torch.empty((B, Lq, Hq, HEAD_DIM), dtype=q.dtype, device=q.device)
    elif out.shape != (B, Lq, Hq, HEAD_DIM) or out.dtype != q.dtype:
        raise ValueError(f"out must be [{B}, {Lq}, {Hq}, {HEAD_DIM}] of {q.dtype}")
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
        if t.stride(-1) != 1:
            raise ValueError(f"{name} needs a unit channel stride")
    strides = np.array([[q.stride(0), q.stride(1), q.stride(2)],
                        [k.stride(0), k.stride(1), k.stride(2)],
                        [v.stride(0), v.stride(1), v.stride(2)],
                        [out.stride(0), out.stride(2), out.stride(1)]], dtype=np.int64)
    base = strides.ctypes.data
    code = dtype_code(q.dtype)
    # Room for the key-split partials where a short call splits (decode-like
    # steps, a short last chunk).
    nbytes = lib.hc_prefill_workspace_bytes(code, B, Hq, Hkv, Lq, Lk)
    # Per-call scratch from the caching allocator (stream-ordered reuse).
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
    if stat_out is None:
        _lib.check(lib.hc_prefill_attn(code, _ptr(q), base, _ptr(k), base + 24, _ptr(v), base + 48, _ptr(out),
                                       base + 72, B, Hq, Hkv, Lq, Lk, float(scale), _ptr(ws), ws.numel(),
                                       _stream(stream, q)))
        return out
    _require_cuda(stat_out)
    if (stat_out.dim() != 4 or tuple(stat_out.shape[:2]) != (B, Hq) or stat_out.shape[3] != 2
            or stat_out.dtype != torch.float32 or not stat_out.is_contiguous()):
        raise ValueError(f"stat_out must be a contiguous float32 tensor of [{B}, {Hq}, W, 2]")
    _lib.check(lib.hc_prefill_attn_stats(code, _ptr(q), base, _ptr(k), base + 24, _ptr(v), base + 48, _ptr(out),
                                         base + 72, B, Hq, Hkv, Lq, Lk, float(scale), _ptr(ws), ws.numel(),
                                         stat_out.shape[2], _ptr(stat_out), _stream(stream, q)))
    return out


# Per-(batch, head) element offsets of gather_rows depend only on shapes and
# strides: built and copied to the device once per layout.
_ROW_OFFSETS = {}


def _row_offsets(B, H, src_strides, dst_strides, device):
    key = (str(device), B, H, tuple(src_strides[:2]), tuple(dst_strides[:2]))
    hit = _ROW_OFFSETS.get(key)
    if hit is None:
        if len(_ROW_OFFSETS) >= 256:
            _ROW_OFFSETS.clear()
        bh = np.arange(B * H, dtype=np.int64)
        hit = _ROW_OFFSETS[key] = (to_device((bh // H) * src_strides[0] + (bh % H) * src_strides[1], device),
                                   to_device((bh // H) * dst_strides[0] + (bh % H) * dst_strides[1], device))
    return hit


def gather_rows(src_k, src_v, idx, counts, dst_k=None, dst_v=None, stream=None):
    """dst[b, h, t] = src[b, h, idx[b*H + h, t]] for t < counts[b*H + h].

    src: [B, H, L, 128] (unit channel stride, any other strides); idx: int32
    [B*H, width] device tensor of source positions (clamped into [0, L));
    counts: int32 [B*H] device tensor or a python int for every job.  The
    destinations default to new [B, H, width, 128] tensors.
    """
    lib = _lib.load()
    _require_cuda(src_k, src_v, idx)
    if src_k.dim() != 4 or src_k.shape[-1] != HEAD_DIM or src_k.stride(-1) != 1 or src_v.shape != src_k.shape:
        raise ValueError("sources must be [B, H, L, 128] with unit channel stride")
    if src_k.stride() != src_v.stride():
        raise ValueError("K and V sources must share strides")
    B, H, L, D = src_k.shape
    if idx.dtype != torch.int32 or idx.dim() != 2 or idx.shape[0] != B * H or idx.stride(1) != 1:
        raise ValueError(f"idx must be int32 [{B * H}, width] with unit inner stride")
    width = idx.shape[1]
    if dst_k is None:
        dst_k = torch.empty((B, H, width, D), dtype=src_k.dtype, device=src_k.device)
        dst_v = torch.empty_like(dst_k)
    if dst_k.shape != (B, H, width, D) or dst_v.shape != dst_k.shape or dst_k.stride() != dst_v.stride() \
            or dst_k.stride(-1) != 1:
        raise ValueError(f"destinations must be [{B}, {H}, {width}, 128] sharing strides")
    if not torch.is_tensor(counts):
        counts = torch.full((B * H,), int(counts), dtype=torch.int32, device=src_k.device)
    if counts.dtype != torch.int32 or counts.numel() != B * H:
        raise ValueError("counts must be int32 [B*H]")
    if width == 0 or B * H == 0:
        return dst_k, dst_v
    src_off, dst_off = _row_offsets(B, H, src_k.stride(), dst_k.stride(), src_k.device)
    _lib.check(lib.hc_gather_rows(dtype_code(src_k.dtype), _ptr(src_k), _ptr(src_v), _ptr(src_off), src_k.stride(2), L,
                                  _ptr(idx), idx.stride(0), _ptr(dst_k), _ptr(dst_v), _ptr(dst_off), dst_k.stride(2),
                                  _ptr(counts), B * H, width, _stream(stream, src_k)))
    return dst_k, dst_v


def append(k_new, v_new, kstore, vstore, row_tile_off, row_len, row_cap, status=None, stream=None):
    """Write k_new/v_new [rows, 128] at slot row_len[r] of every row, then row_len += 1."""
    lib = _lib.load()
    _require_cuda(k_new, v_new, kstore, vstore, row_tile_off, row_len, row_cap, status)
    rows = row_len.numel()
    if k_new.shape != (rows, HEAD_DIM) or v_new.shape != (rows, HEAD_DIM):
        raise ValueError(f"new k/v must be [{rows}, {HEAD_DIM}]")
    k_new = k_new.contiguous()
    v_new = v_new.contiguous()
    _lib.check(lib.hc_append(dtype_code(kstore.dtype), _ptr(k_new), _ptr(v_new), HEAD_DIM, _ptr(kstore),
                             _ptr(vstore), _ptr(row_tile_off), _ptr(row_len), _ptr(row_cap), rows, _ptr(status),
                             _stream(stream, kstore)))


def store_read(kstore, vstore, row_tile_off, rows_sel, count, stream=None):
    """Natural-layout copy [len(rows_sel), count, 128] of store slots [0, count)."""
    lib = _lib.load()
    _require_cuda(kstore, vstore, row_tile_off)
    rows_sel = torch.as_tensor(rows_sel, dtype=torch.int32, device=kstore.device)
    n = rows_sel.numel()
    dk = torch.empty((n, count, HEAD_DIM), dtype=kstore.dtype, device=kstore.device)
    dv = torch.empty_like(dk)
    _lib.check(lib.hc_store_read(dtype_code(kstore.dtype), _ptr(kstore), _ptr(vstore), _ptr(row_tile_off),
                                 _ptr(rows_sel), n, int(count), _ptr(dk), _ptr(dv), _stream(stream, kstore)))
    return dk, dv


def score(q, q_off, q_head_stride, q_row_stride, k, k_off, k_tok_stride, seq_len, group, window, span, pooling,
          kernel, scale, flags=0, row_tile_off=None, k_row=None, out=None, hist=None, stream=None):
    """Pooled window scores [jobs, W', span] (see hc_score in include/hc.h).

    q / k are the base tensors; q_off / k_off are int64 device tensors of
    per-job element offsets (k_off unused when reading a tiled store through
    row_tile_off / k_row).  hist: optional uint32-sized int32 tensor of
    [jobs * W', HIST_BINS] that receives each score row's first-digit key
    histogram (for drift_select).
    """
    lib = _lib.load()
    _require_cuda(q, k, q_off, k_off, row_tile_off, k_row)
    if q.dtype != k.dtype:
        raise TypeError("q and k must share a dtype")
    njobs = q_off.numel()
    wout = 1 if flags & _lib.HC_SCORE_SUM_WINDOW else window
    if out is None:
        out = torch.empty((njobs, wout, span), dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or out.numel() < njobs * wout * span or not out.is_contiguous():
        raise ValueError("out must be a contiguous float32 tensor of [jobs, W', span]")
    if q_off.dtype != torch.int64 or (k_off is not None and k_off.dtype != torch.int64):
        raise TypeError("offsets must be int64")
    if k_row is not None and k_row.dtype != torch.int32:
        raise TypeError("k_row must be int32")
    if hist is not None:
        _require_cuda(hist)
        if hist.dtype != torch.int32 or not hist.is_contiguous() or hist.numel() < njobs * wout * HIST_BINS:
            raise ValueError(f"hist must be a contiguous int32 tensor of [jobs * W', {HIST_BINS}]")
    nbytes = lib.hc_score_workspace_size(njobs, seq_len, group, window, flags)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    pool = {"avgpool": 0, "maxpool": 1}[pooling] if isinstance(pooling, str) else int(pooling)
    _lib.check(lib.hc_score(dtype_code(q.dtype), _ptr(q), _ptr(q_off), int(q_head_stride), int(q_row_stride), _ptr(k),
                            _ptr(k_off), int(k_tok_stride), _ptr(row_tile_off), _ptr(k_row), njobs, int(seq_len),
                            int(group), int(window), int(flags), int(span), pool, int(kernel), float(scale),
                            _ptr(out), _ptr(ws), ws.numel(), _ptr(hist), _stream(stream, q)))
    return out


def score_with_stats(q, q_off, q_head_stride, q_row_stride, k, k_off, k_tok_stride, seq_len, group, window, span,
                     pooling, kernel, scale, stats, stat_off=None, stat_head_stride=0, flags=0, row_tile_off=None,
                     k_row=None, out=None, stream=None):
    """ops.score with each query row's softmax statistics given (one key pass,
    no rounding flags): row r = g*window + w of job j reads (M, L) at
    stats[base + 2r], or stats[base + g*stat_head_stride + 2w] with a
    nonzero head stride, base = stat_off[j] (or 2*group*window*j without
    stat_off).  See hc_score_with_stats in include/hc.h."""
    lib = _lib.load()
    _require_cuda(q, k, q_off, k_off, row_tile_off, k_row, stats, stat_off)
    if q.dtype != k.dtype:
        raise TypeError("q and k must share a dtype")
    if q_off.dtype != torch.int64 or (k_off is not None and k_off.dtype != torch.int64):
        raise TypeError("offsets must be int64")
    if stat_off is not None and stat_off.dtype != torch.int64:
        raise TypeError("stat_off must be int64")
    if stats.dtype != torch.float32:
        raise TypeError("stats must be float32")
    njobs = q_off.numel()
    wout = 1 if flags & _lib.HC_SCORE_SUM_WINDOW else window
    if out is None:
        out = torch.empty((njobs, wout, span), dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or out.numel() < njobs * wout * span or not out.is_contiguous():
        raise ValueError("out must be a contiguous float32 tensor of [jobs, W', span]")
    ws = torch.empty(max(njobs * wout * group * span * 4, 256), dtype=torch.uint8, device=q.device)
    pool = {"avgpool": 0, "maxpool": 1}[pooling] if isinstance(pooling, str) else int(pooling)
    _lib.check(lib.hc_score_with_stats(dtype_code(q.dtype), _ptr(q), _ptr(q_off), int(q_head_stride),
                                       int(q_row_stride), _ptr(k), _ptr(k_off), int(k_tok_stride), _ptr(row_tile_off),
                                       _ptr(k_row), njobs, int(seq_len), int(group), int(window), int(flags),
                                       int(span), pool, int(kernel), float(scale), _ptr(stats), _ptr(stat_off),
                                       int(stat_head_stride), _ptr(out), _ptr(ws), ws.numel(), _stream(stream, q)))
    return out


def score_given_stats(q, q_off, q_head_stride, q_row_stride, kstore, row_tile_off, k_row, seq_len, group, window,
                      pooling, kernel, scale, stats, stat_off, out=None, stream=None, flags=0):
    """Pivot drift scores [jobs, window, seq_len] in one pass over the keys of
    store rows k_row, given each query row's softmax statistics (M, L) at
    stats[stat_off[j] + 2r] (hc_score_given_stats in include/hc.h); flags
    HC_SCORE_ROUND_BF16 / _F16 apply the reference's cast chain, with
    statistics of that chain (decode_attn's stat_flags)."""
    lib = _lib.load()
    _require_cuda(q, kstore, q_off, row_tile_off, k_row, stats, stat_off)
    if q.dtype != kstore.dtype:
        raise TypeError("q and the store must share a dtype")
    if q_off.dtype != torch.int64 or stat_off.dtype != torch.int64 or k_row.dtype != torch.int32:
        raise TypeError("q_off / stat_off must be int64 and k_row int32")
    if stats.dtype != torch.float32:
        raise TypeError("stats must be float32")
    njobs = q_off.numel()
    if out is None:
        out = torch.empty((njobs, window, seq_len), dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or out.numel() < njobs * window * seq_len or not out.is_contiguous():
        raise ValueError("out must be a contiguous float32 tensor of [jobs, window, seq_len]")
    pool = {"avgpool": 0, "maxpool": 1}[pooling] if isinstance(pooling, str) else int(pooling)
    _lib.check(lib.hc_score_given_stats(dtype_code(q.dtype), _ptr(q), _ptr(q_off), int(q_head_stride),
                                        int(q_row_stride), _ptr(kstore), _ptr(row_tile_off), _ptr(k_row), njobs,
                                        int(seq_len), int(group), int(window), int(flags), pool, int(kernel),
                                        float(scale),
                                        _ptr(stats), _ptr(stat_off), _ptr(out), _stream(stream, q)))
    return out


def cake_score(q, q_off, q_head_stride, q_row_stride, k, k_off, k_tok_stride, batch, kv_heads, seq_len, group,
               window, scale, gamma, flags=0, out=None, stats=None, stream=None):
    """CAKE scores [batch * kv_heads, seq_len - window] and the float32 device
    triple (entropy, variance sum, preference) (see hc_cake_score in
    include/hc.h).  q_off / k_off: int64 device tensors of per-job offsets."""
    lib = _lib.load()
    _require_cuda(q, k, q_off, k_off)
    if q.dtype != k.dtype:
        raise TypeError("q and k must share a dtype")
    if q_off.dtype != torch.int64 or k_off.dtype != torch.int64:
        raise TypeError("offsets must be int64")
    njobs, span = batch * kv_heads, seq_len - window
    if q_off.numel() != njobs or k_off.numel() != njobs:
        raise ValueError(f"expected {njobs} job offsets")
    if out is None:
        out = torch.empty((njobs, max(span, 0)), dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or out.numel() < njobs * span or not out.is_contiguous():
        raise ValueError("out must be a contiguous float32 tensor of [jobs, span]")
    if stats is None:
        stats = torch.empty(3, dtype=torch.float32, device=q.device)
    nbytes = lib.hc_cake_workspace_size(batch, kv_heads, seq_len, group, window)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    _lib.check(lib.hc_cake_score(dtype_code(q.dtype), _ptr(q), _ptr(q_off), int(q_head_stride), int(q_row_stride),
                                 _ptr(k), _ptr(k_off), int(k_tok_stride), int(batch), int(kv_heads), int(seq_len),
                                 int(group), int(window), int(flags), float(scale), float(gamma), _ptr(out),
                                 _ptr(stats), _ptr(ws), ws.numel(), _stream(stream, q)))
    return out, stats


def select_topk(scores, caps, span, window=0, idx=None, counts=None, stream=None, key_bits=0):
    """Ascending kept positions per job: scores [jobs, >= span] float32, caps int32 [jobs].
    key_bits: see hc_select_topk (KEY_BITS[round dtype] for cast-chain scores)."""
    lib = _lib.load()
    _require_cuda(scores, caps, idx, counts)
    if scores.dtype != torch.float32 or scores.dim() != 2 or scores.stride(1) != 1:
        raise ValueError("scores must be float32 [jobs, n] with unit stride")
    if caps.dtype != torch.int32:
        raise TypeError("caps must be int32")
    njobs = scores.shape[0]
    if idx is None:
        idx = torch.empty((njobs, span + window), dtype=torch.int32, device=scores.device)
    if counts is None:
        counts = torch.empty(njobs, dtype=torch.int32, device=scores.device)
    hist = SELECT_HIST.get(scores.device, lib.hc_select_hist_size(njobs))
    scratch = torch.empty(max(lib.hc_select_scratch_size(njobs, int(span)), 16), dtype=torch.uint8,
                          device=scores.device)
    _lib.check(lib.hc_select_topk(_ptr(scores), scores.stride(0), njobs, int(span), _ptr(caps), int(window), _ptr(idx),
                                  idx.stride(0), _ptr(counts), _ptr(hist), hist.numel(), _ptr(scratch),
                                  scratch.numel(), int(key_bits), _stream(stream, scores)))
    return idx, counts


def drift_select(scores, caps, K, bits, nbits, trig_of, nlead, batch, steps, threshold, trigger, hist, overlap=None,
                 stream=None):
    """Drift decision of sets j = leader * batch + b from their step scores
    (scores [sets * steps, >= nbits] float32, row j * steps + s, with the
    first-digit key histograms `hist` that score() built for them, or None
    to build them here): per step
    the overlap of its top-K with bits[j] (out: overlap [sets * steps] int32),
    trigger[leader] = median over steps of the batch-mean overlap / K <
    threshold, and bits[j] := top-K of the last step where trigger[trig_of[j]]."""
    lib = _lib.load()
    _require_cuda(scores, caps, bits, trig_of, trigger, overlap, hist)
    if scores.dtype != torch.float32 or scores.dim() != 2 or scores.stride(1) != 1:
        raise ValueError("scores must be float32 [jobs, n] with unit stride")
    for name, t in (("caps", caps), ("bits", bits), ("trig_of", trig_of), ("trigger", trigger), ("hist", hist)):
        if t is not None and t.dtype != torch.int32:
            raise TypeError(f"{name} must be int32")
    njobs = scores.shape[0]
    if njobs % steps or caps.numel() < njobs:
        raise ValueError("scores rows must be sets x steps, with one cap per row")
    nsets = njobs // steps
    if bits.dim() != 2 or bits.shape[0] < nsets or trig_of.numel() < nsets:
        raise ValueError("one bitmask set and one leader index per set")
    if hist is not None and (not hist.is_contiguous() or hist.numel() < njobs * HIST_BINS):
        raise ValueError(f"hist must be a contiguous int32 tensor of [jobs, {HIST_BINS}]")
    if overlap is None:
        overlap = torch.empty(njobs, dtype=torch.int32, device=scores.device)
    scratch = torch.empty(max(lib.hc_drift_scratch_size(njobs, int(nbits)), 16), dtype=torch.uint8,
                          device=scores.device)
    _lib.check(lib.hc_drift_select(_ptr(scores), scores.stride(0), nsets, int(steps), int(batch), int(nbits),
                                   _ptr(caps), int(K), _ptr(bits), bits.stride(0), _ptr(trig_of), int(nlead),
                                   float(threshold), _ptr(overlap), _ptr(trigger), _ptr(hist), _ptr(scratch),
                                   scratch.numel(), _stream(stream, scores)))
    return overlap


def set_bits(idx, counts, bits, nbits, fixed_count=0, trigger=None, trig_of=None, stream=None, row_of=None):
    """bits[j] = set of the first counts[j] (or fixed_count) positions of idx[r]
    (cleared first), r = row_of[j] (int64 device tensor, one valid row of idx
    per set) or j."""
    lib = _lib.load()
    _require_cuda(idx, counts, bits, trigger, trig_of, row_of)
    if idx.dtype != torch.int32 or bits.dtype != torch.int32 or idx.dim() != 2 or bits.dim() != 2:
        raise TypeError("idx and bits must be 2-D int32 tensors")
    if row_of is not None and row_of.dtype != torch.int64:
        raise TypeError("row_of must be int64")
    nsets = idx.shape[0] if row_of is None else row_of.numel()
    if bits.shape[0] < nsets:
        raise ValueError("one bitmask row per set")
    _lib.check(lib.hc_set_bits(_ptr(idx), idx.stride(0), _ptr(counts), int(fixed_count), nsets, _ptr(bits),
                               bits.stride(0), int(nbits), _ptr(trigger), _ptr(trig_of), _ptr(row_of),
                               _stream(stream, bits)))


def overlap_count(idx, count, bits, nbits, ref_of=None, out=None, stream=None):
    """|first `count` positions of idx[j]  ∩  bits[ref_of[j]]| per list j."""
    lib = _lib.load()
    _require_cuda(idx, bits, ref_of, out)
    if out is None:
        out = torch.empty(idx.shape[0], dtype=torch.int32, device=idx.device)
    _lib.check(lib.hc_overlap_count(_ptr(idx), idx.stride(0), int(count), idx.shape[0], _ptr(bits), bits.stride(0),
                                    int(nbits), _ptr(ref_of), _ptr(out), _stream(stream, bits)))
    return out


def drift_decide(counts, npiv, batch, steps, K, threshold, trigger, overlap=None, median=None, stream=None):
    """Per pivot: batch-mean overlap per step, median over steps, trigger = median < threshold."""
    lib = _lib.load()
    _require_cuda(counts, trigger, overlap, median)
    _lib.check(lib.hc_drift_decide(_ptr(counts), int(npiv), int(batch), int(steps), int(K), float(threshold),
                                   _ptr(overlap), _ptr(median), _ptr(trigger), _stream(stream, counts)))
