"""State-dict fixtures as plain data: a JSON skeleton plus named arrays.

``encode(obj)`` walks an optimizer ``state_dict()`` (nested dicts, lists,
tuples, tensors, torch dtypes, Python scalars) and returns ``(skeleton,
arrays)``: ``skeleton`` is JSON text in which every tensor is replaced by a
reference ``{"__tensor__": name, "dtype": ..., "shape": [...]}`` and
``arrays`` maps those names to numpy arrays (bf16 and fp16 stored as their
uint16 bit patterns).  ``decode(skeleton, arrays)`` rebuilds the same
structure with CPU tensors of the original dtypes, so a checkpoint written
by one optimizer can be stored in an ``.npz`` fixture and loaded into another
without pickling anything.
"""

import json

import numpy as np
import torch

_DTYPES = {
    "float32": torch.float32, "float64": torch.float64, "bfloat16": torch.bfloat16, "float16": torch.float16,
    "int8": torch.int8, "uint8": torch.uint8, "int16": torch.int16, "int32": torch.int32, "int64": torch.int64,
    "bool": torch.bool,
}
_NAMES = {v: k for k, v in _DTYPES.items()}


def _to_np(t):
    # a copy: state_dict() hands out the live state tensors, which later steps update in place
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def _from_np(a, dtype, shape):
    if dtype in (torch.bfloat16, torch.float16):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype).reshape(shape).clone()
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).reshape(shape).clone()


def encode(obj, prefix="t"):
    arrays = {}

    def enc(x):
        if torch.is_tensor(x):
            name = f"{prefix}{len(arrays)}"
            arrays[name] = _to_np(x)
            return {"__tensor__": name, "dtype": _NAMES[x.dtype], "shape": list(x.shape)}
        if isinstance(x, torch.dtype):
            return {"__dtype__": _NAMES[x]}
        if isinstance(x, dict):
            return {"__dict__": [[enc(k), enc(v)] for k, v in x.items()]}
        if isinstance(x, tuple):
            return {"__tuple__": [enc(v) for v in x]}
        if isinstance(x, list):
            return [enc(v) for v in x]
        if x is None or isinstance(x, (bool, int, float, str)):
            return x
        raise TypeError(f"cannot encode {type(x)}")

    return json.dumps(enc(obj)), arrays


def decode(skeleton, arrays):
    def dec(x):
        if isinstance(x, dict):
            if "__tensor__" in x:
                return _from_np(arrays[x["__tensor__"]], _DTYPES[x["dtype"]], tuple(x["shape"]))
            if "__dtype__" in x:
                return _DTYPES[x["__dtype__"]]
            if "__dict__" in x:
                return {dec(k): dec(v) for k, v in x["__dict__"]}
            if "__tuple__" in x:
                return tuple(dec(v) for v in x["__tuple__"])
            raise ValueError(f"unknown node {sorted(x)}")
        if isinstance(x, list):
            return [dec(v) for v in x]
        return x

    return dec(json.loads(skeleton))
