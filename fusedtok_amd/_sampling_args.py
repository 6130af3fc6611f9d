"""Host-side argument normalisation of the sampling ops.

The samplers take Python-level arguments that have to become device
vectors: one seed per row, and each row's token history for the
repetition penalty. Histories arrive in three forms (reference
``__init__.py:2415-2481``): ragged per-row sequences, a 2-D array whose rows
are all used, or flat ids with row offsets. All three become one flat int64
vector plus rows + 1 offsets (a CSR layout), which is what the kernels read.

Contract (the reference's, ``__init__.py:322-395``): host-origin ids are
range-checked against the vocabulary; a GPU id tensor is trusted (the
kernels drop out-of-range entries). Seeds are unsigned 64-bit patterns
accepted in [0, 2**63). Non-integer inputs are TypeErrors, shapes and
ranges ValueErrors.
"""

import numpy as np
import torch


def check_params(p, temperature, penalty=1.0):
    if not penalty > 0.0:
        raise ValueError("penalty must be > 0")
    if not 0.0 < p <= 1.0:
        raise ValueError("p must be in (0, 1]")
    if not temperature > 0.0:
        raise ValueError("temperature must be > 0")


def _host(x):
    """Any array-like (list, numpy, torch on any device) as numpy."""
    if torch.is_tensor(x):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def _require_ints(a, what):
    if a.size and a.dtype.kind not in "iu":
        raise TypeError(f"{what} must hold integer values (got dtype {a.dtype})")


def seed_vector(seeds, rows):
    """One int64 seed per row: None gives 0 .. rows - 1."""
    if seeds is None:
        return np.arange(rows, dtype=np.int64)
    a = _host(seeds)
    if a.dtype.kind not in "iu":
        raise TypeError("seeds must contain integers")
    if a.ndim != 1:
        raise ValueError("seeds must be 1-D")
    if len(a) != rows:
        raise ValueError("seeds must have one entry per row")
    too_big = a.dtype.kind == "u" and a.size and int(a.max()) >= 1 << 63
    negative = a.dtype.kind == "i" and a.size and int(a.min()) < 0
    if too_big or negative:
        raise ValueError("seeds values must be in [0, 2**63)")
    return a.astype(np.int64)


def history_1d(ids, vocab, device):
    """One row's token history: a trusted GPU tensor passes through as int64
    (device tensors are never read back); host values are checked against
    [0, vocab) and returned as numpy int64, or uploaded when `device` is
    given."""
    if torch.is_tensor(ids) and ids.is_cuda:
        if ids.ndim != 1:
            raise ValueError("sampled_ids must be 1-D")
        return ids.to(torch.int64).contiguous()
    a = _host(ids)
    _require_ints(a, "sampled_ids")
    if a.ndim != 1:
        raise ValueError("sampled_ids must be 1-D")
    a = a.astype(np.int64)
    if a.size and not (0 <= int(a.min()) and int(a.max()) < vocab):
        raise ValueError(f"sampled_ids values must be in [0, {vocab})")
    return a if device is None else torch.from_numpy(a).to(device)


def histories_csr(sampled_ids, ids_offsets, rows, vocab):
    """Per-row histories in any accepted form -> (flat int64 ids, int64
    offsets with rows + 1 entries), host side and range-checked."""
    if ids_offsets is not None:
        flat, offs = _host(sampled_ids), _host(ids_offsets)
        if flat.ndim != 1:
            raise ValueError("sampled_ids with ids_offsets must be a flat 1-D array")
        if offs.ndim != 1 or offs.size != rows + 1:
            raise ValueError("ids_offsets must be 1-D with rows + 1 entries")
        if flat.size and flat.dtype.kind not in "iu":
            raise TypeError("sampled_ids entries must be integers")
        if offs.size and offs.dtype.kind not in "iu":
            raise TypeError("ids_offsets entries must be integers")
        flat, offs = flat.astype(np.int64), offs.astype(np.int64)
        steps = np.diff(offs)
        if offs[0] != 0 or offs[-1] != flat.size or (steps < 0).any():
            raise ValueError("ids_offsets must start at 0, end at len(sampled_ids) "
                             "and be non-decreasing")
    elif isinstance(sampled_ids, (list, tuple)):
        if len(sampled_ids) != rows:
            raise ValueError("sampled_ids must have one entry per row")
        parts = [_host(r).reshape(-1) for r in sampled_ids]
        for part in parts:
            if part.size and part.dtype.kind not in "iu":
                raise TypeError("sampled_ids entries must be integers")
        lengths = np.array([part.size for part in parts], dtype=np.int64)
        offs = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
        flat = (np.concatenate([part.astype(np.int64) for part in parts])
                if parts else np.zeros(0, np.int64))
    else:
        grid = _host(sampled_ids)
        if grid.ndim != 2:
            raise ValueError("sampled_ids must be per-row sequences, a 2-D array, "
                             "or flat ids plus ids_offsets")
        if grid.shape[0] != rows:
            raise ValueError("sampled_ids must have one entry per row")
        if grid.size and grid.dtype.kind not in "iu":
            raise TypeError("sampled_ids entries must be integers")
        flat = grid.astype(np.int64).reshape(-1)
        offs = grid.shape[1] * np.arange(rows + 1, dtype=np.int64)
    if flat.size and (int(flat.min()) < 0 or int(flat.max()) >= vocab):
        raise ValueError(f"sampled_ids values must be in [0, {vocab})")
    return np.ascontiguousarray(flat), np.ascontiguousarray(offs)


# Small per-call int64 vectors (histories, offsets, seeds) are staged in a
# ring of pinned host buffers. The kernels read them in place through the
# buffer's device mapping (no copy on the stream: an asynchronous copy's
# completion reached the compute queue only tens of microseconds after the
# kernels were queued); where the runtime reports no mapping, one
# non-blocking copy per call takes them up instead. A slot is refilled only
# after the work that read it has completed (its event). A pageable copy
# per vector made every call wait for the GPU to drain. Above IN_PLACE_MAX
# values (long histories) the slot is uploaded too: each of a row's slices
# reads the row's history, so in-place reads would cross PCIe once per
# slice (64 rows x 8 slices x 8k ids is 32 MB of scattered reads). The
# bound counts the whole slot (ids, offsets, seeds): 64 rows of 64 ids with
# their offsets and seeds (4225 values) stay in place (decode_step_batched
# at 64 x 128256: 87.7 us in place, 94.5 us uploaded).
IN_PLACE_MAX = 8192


class _PinnedRing:
    def __init__(self, slots=4):
        self.slots = [[None, None, 0] for _ in range(slots)]  # [buffer, event, device address]
        self.turn = 0

    def _fill(self, arrays, mapper=None):
        sizes = [int(a.size) for a in arrays]
        total = max(1, sum(sizes))
        slot = self.slots[self.turn % len(self.slots)]
        self.turn += 1
        buf, done = slot[0], slot[1]
        if done is not None:
            done.synchronize()
        if buf is None or buf.numel() < total:
            grow = max(total, 1024, 0 if buf is None else 2 * buf.numel())
            buf = torch.empty(grow, dtype=torch.int64, pin_memory=True)
            slot[0], slot[2] = buf, (mapper(buf.data_ptr()) if mapper else 0)
        view = buf.numpy()
        bounds = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
        for a, lo, hi in zip(arrays, bounds[:-1], bounds[1:]):
            view[lo:hi] = a.reshape(-1)
        return slot, total, bounds

    def launch_in_place(self, arrays, device, mapper, launch):
        """launch(addresses): the vectors' device-accessible addresses
        (int), read in place from pinned host memory when `mapper` gives the
        buffer a device address, else from an uploaded copy. The slot's
        event follows the launch on the current stream."""
        slot, total, bounds = self._fill(arrays, mapper)
        base = slot[2]
        if base and total <= IN_PLACE_MAX:
            launch([base + 8 * int(lo) for lo in bounds[:-1]])
        else:  # no device mapping, or long vectors: one copy of the slot
            dev = torch.empty(total, dtype=torch.int64, device=device)
            dev.copy_(slot[0][:total], non_blocking=True)
            launch([dev.data_ptr() + 8 * int(lo) for lo in bounds[:-1]])
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(device))
        slot[1] = ev


_RING = _PinnedRing()


def launch_with_int64(arrays, device, mapper, launch):
    """Host int64 numpy vectors staged for one launch: launch(addresses)
    gets device-accessible addresses of them (pinned host memory read in
    place, or an uploaded copy); `mapper(host_ptr)` returns the device
    address of pinned host memory or 0."""
    _RING.launch_in_place(arrays, device, mapper, launch)
