"""Argument contracts of the public ops, stated as data.

An op declares its operands once, as a :class:`Contract`:

- :class:`Arr` is an array operand. It has a symbolic shape (``"B Hq D"``;
  ``"rows? cols"`` allows a missing leading dimension, ``"=k_pool"`` copies
  another operand's shape, ``"*"`` is any shape) and the element types it
  accepts. It may have to share another operand's element type, it may be
  written in place, and it may be converted to float32 / made contiguous
  instead of rejected (norm weights, per-channel scales).
- :class:`Idx` is an integer operand that indexes the caches (lengths,
  block tables). Host-origin values are range-checked; device-resident
  values are trusted and never read back.
- :class:`Rule` is a condition over the bound shape symbols and the
  call's scalar arguments, with the exception it raises.

:meth:`Contract.bind` checks one call against its contract and returns a
:class:`Call`: the operands (device tensors, or host arrays on the staged
path) and the shape symbols as attributes. :meth:`Call.staged` runs the
same op on the GPU for host operands: it uploads them, calls the op again,
and brings results and in-place operands back. An op body is therefore
written once, for device tensors, and its checks live in its contract.

Error classes follow the reference's contract (reference
``python/fusedtok/__init__.py:112-182``): TypeError for element types and
device families, ValueError for shapes and values, RuntimeError when a host
call finds no device.
"""

import numpy as np
import torch

FLOATS = (torch.float32, torch.bfloat16, torch.float16)
INT8 = (torch.int8,)


def dtype_names(dtypes):
    return ", ".join(str(d).replace("torch.", "") for d in dtypes)


class Arr:
    """An array operand of a contract (see the module docstring)."""

    def __init__(self, name, shape="*", dtypes=FLOATS, *, same_dtype=None,
                 optional=False, inplace=False, upcast=False, mismatch=None,
                 rank_msg=None, dtype_msg=None):
        self.name = name
        self.rank_msg = rank_msg
        self.shape = shape
        self.dtypes = dtypes
        self.same_dtype = same_dtype
        self.optional = optional
        self.inplace = inplace
        self.upcast = upcast
        self.mismatch = mismatch
        self.dtype_msg = dtype_msg

    # -- device operands ----------------------------------------------------
    def on_device(self, t):
        if not (torch.is_tensor(t) and t.is_cuda):
            raise TypeError(f"{self.name} must be a GPU tensor when the primary "
                            "input is on the GPU")
        if self.upcast:
            if t.dtype is not self.dtypes[0]:
                t = t.to(self.dtypes[0])
            return t.contiguous()
        if t.dtype not in self.dtypes:
            raise TypeError(self.dtype_msg or
                            f"{self.name} must be one of ({dtype_names(self.dtypes)}), "
                            f"got {t.dtype}")
        if not t.is_contiguous():
            raise ValueError(f"{self.name} must be contiguous")
        return t

    # -- host operands ------------------------------------------------------
    def on_host(self, x):
        if torch.is_tensor(x) and x.is_cuda:
            raise TypeError(f"{self.name} is a GPU tensor while another input is "
                            "host-side; move all inputs to the same device")
        want = torch.int8 if self.dtypes == INT8 else torch.float32
        if self.inplace:
            raw = x.numpy() if torch.is_tensor(x) else x
            if not (isinstance(raw, np.ndarray) and raw.dtype == np.float32
                    and raw.flags["C_CONTIGUOUS"]):
                raise TypeError(f"{self.name} must be a float32 C-contiguous array "
                                "(in-place op; conversion would drop writes)")
            return raw
        if want is torch.int8:
            a = x.detach().numpy() if torch.is_tensor(x) else np.asarray(x)
            if a.size and not np.issubdtype(a.dtype, np.integer):
                raise TypeError(self.dtype_msg or
                                f"{self.name} must be an integer array, got {a.dtype}")
            return np.ascontiguousarray(a, dtype=np.int8)
        if torch.is_tensor(x):
            x = x.detach().to(torch.float32).numpy()
        return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


class Idx:
    """An integer operand addressing the caches (module docstring).

    ``shape`` binds symbols like an :class:`Arr`; ``bound(call)`` is the
    largest allowed value, inclusive unless ``open_bound``; ``what`` names
    the shape in the error message."""

    def __init__(self, name, shape, bound, *, open_bound=False, optional=False,
                 what=None):
        self.name = name
        self.shape = shape
        self.bound = bound
        self.open_bound = open_bound
        self.optional = optional
        self.what = what

    def host_values(self, x):
        """Host-origin values as an int numpy array; None for a GPU tensor."""
        if torch.is_tensor(x):
            if x.is_cuda:
                return None
            x = x.detach().cpu().numpy()
        a = np.asarray(x)
        if a.size and not np.issubdtype(a.dtype, np.integer):
            raise TypeError(f"{self.name} must hold integer values (got dtype {a.dtype})")
        return np.ascontiguousarray(a, dtype=np.int32)

    def check_range(self, a, call):
        hi = self.bound(call)
        if not a.size:
            return
        lo_bad = int(a.min()) < 0
        hi_bad = int(a.max()) >= hi if self.open_bound else int(a.max()) > hi
        if lo_bad or hi_bad:
            close = ")" if self.open_bound else "]"
            raise ValueError(f"{self.name} entries must be in [0, {hi}{close}")


class Rule:
    """``test(call)`` must hold; otherwise ``exc(message)`` is raised."""

    def __init__(self, test, message, exc=ValueError):
        self.test = test
        self.message = message
        self.exc = exc


def _parse(shape):
    if shape == "*" or shape.startswith("="):
        return shape
    return tuple(shape.split())


class Call:
    """One checked call: operands and shape symbols as attributes."""

    def __init__(self, contract, values, device):
        self._contract = contract
        self._values = values
        self._primary = values[contract.operands[0].name]
        self.device = device
        self.dims = {}
        for k, v in values.items():
            setattr(self, k, v)

    def __getattr__(self, name):
        dims = self.__dict__.get("dims", {})
        if name in dims:
            return dims[name]
        raise AttributeError(name)

    @property
    def on_gpu(self):
        return self.device is not None

    def ptr(self, name):
        v = getattr(self, name)
        return None if v is None else v.data_ptr()

    def staged(self, op):
        """Run `op` on the GPU for this host call: upload every array and
        index operand, call `op` with the device tensors and the same
        scalar arguments, copy in-place operands back into the caller's
        arrays, and return the op's results in the caller's family (numpy,
        or CPU torch when the primary input was a torch tensor)."""
        if not torch.cuda.is_available():
            raise RuntimeError(
                "fusedtok_amd runs on the GPU only: no HIP device is available "
                "for these host inputs (there is no CPU fallback)")
        dev = torch.device("cuda", torch.cuda.current_device())
        args = dict(self._values)
        uploaded = {}
        for spec in self._contract.operands:
            v = args.get(spec.name)
            if v is None:
                continue
            if isinstance(v, np.ndarray):
                uploaded[spec.name] = torch.from_numpy(np.ascontiguousarray(v)).to(dev)
                args[spec.name] = uploaded[spec.name]
        res = op(**args)
        for spec in self._contract.operands:
            if isinstance(spec, Arr) and spec.inplace and spec.name in uploaded:
                np.copyto(self._values[spec.name], uploaded[spec.name].cpu().numpy())
        as_torch = torch.is_tensor(self._primary)

        def back(r):
            if not torch.is_tensor(r):
                return r
            r = r.cpu()
            return r if as_torch else r.numpy()
        if isinstance(res, tuple):
            return tuple(back(r) for r in res)
        return back(res)


class Contract:
    """The operands and rules of one op (module docstring). The first
    operand decides the path: a GPU tensor there means every operand must
    be a GPU tensor (zero copy); otherwise the call is staged."""

    def __init__(self, *operands, rules=(), rank_msg=None, host=True,
                 host_rules=()):
        self.operands = operands
        self.rules = rules
        self.host_rules = host_rules
        self.rank_msg = rank_msg
        self.host = host

    def bind(self, **values):
        primary = values[self.operands[0].name]
        gpu = torch.is_tensor(primary) and primary.is_cuda
        if not gpu and not self.host:
            raise TypeError(f"{self.operands[0].name} must be a GPU tensor (this op "
                            "has no host path)")
        call = Call(self, values, primary.device if gpu else None)
        shapes = {}
        for spec in self.operands:
            v = values.get(spec.name)
            if v is None:
                if not spec.optional:
                    raise TypeError(f"{spec.name} is required")
                continue
            if isinstance(spec, Arr):
                v = spec.on_device(v) if gpu else spec.on_host(v)
                if spec.same_dtype is not None and gpu:
                    other = getattr(call, spec.same_dtype)
                    if v.dtype is not other.dtype:
                        raise TypeError(f"{spec.name} must have the same dtype as "
                                        f"{spec.same_dtype}")
                self._bind_shape(call, spec, tuple(v.shape), shapes)
            else:
                v = self._index(call, spec, v, gpu, shapes)
            setattr(call, spec.name, v)
            call._values[spec.name] = v
        for rule in self.rules + (() if gpu else self.host_rules):
            if not rule.test(call):
                raise rule.exc(rule.message)
        return call

    def _bind_shape(self, call, spec, shape, shapes):
        shapes[spec.name] = shape
        pat = _parse(spec.shape)
        if pat == "*":
            return
        if isinstance(pat, str):  # "=other": the same shape as another operand
            if shape != shapes[pat[1:]]:
                raise ValueError(spec.mismatch or
                                 f"{spec.name} must have the same shape as {pat[1:]}")
            return
        syms = list(pat)
        if syms and syms[0].endswith("?"):
            if len(shape) == len(syms) - 1:
                shape = (1,) + shape
            syms[0] = syms[0][:-1]
        if len(shape) != len(syms):
            raise ValueError(spec.rank_msg or self.rank_msg or spec.mismatch or
                             f"{spec.name} must be {len(syms)}-D")
        for sym, n in zip(syms, shape):
            if sym.isdigit():
                ok = int(sym) == n
            elif sym in call.dims:
                ok = call.dims[sym] == n
            else:
                call.dims[sym] = int(n)
                ok = True
            if not ok:
                raise ValueError(spec.mismatch or
                                 f"{spec.name} has the wrong size in {sym}")

    def _index(self, call, spec, v, gpu, shapes):
        host = spec.host_values(v)
        if host is None:
            if not gpu:
                raise TypeError(f"{spec.name} must be a host array on this path")
            t = v if v.dtype is torch.int32 else v.to(torch.int32)
            t = t.contiguous()
            self._bind_index_shape(call, spec, tuple(t.shape))
            return t
        self._bind_index_shape(call, spec, host.shape)
        spec.check_range(host, call)
        return torch.from_numpy(host).to(call.device) if gpu else host

    def _bind_index_shape(self, call, spec, shape):
        syms = spec.shape.split()
        ok = len(shape) == len(syms)
        if ok:
            for sym, n in zip(syms, shape):
                if sym in call.dims:
                    ok = ok and call.dims[sym] == n
                else:
                    call.dims[sym] = int(n)
        if not ok:
            raise ValueError(spec.what)
