"""GGUF weight parameters of the linear method (reference: quantization/params.py:22-132,
304-434): an uninitialised uint8 `weight` that collects one tensor per loaded shard in
`data_container`, and a `weight_type` parameter that records the ggml type per shard. Tensor-
parallel narrowing is vLLM's and is not restated (one GPU)."""

import torch
from torch.nn.parameter import Parameter, UninitializedParameter


def _gguf_shard_id_as_int(shard_id):
    if isinstance(shard_id, int):
        return shard_id
    return {"q": 0, "k": 1, "v": 2}[shard_id]


def _gguf_ordered_shard_ids(shard_ids):
    return sorted(shard_ids, key=_gguf_shard_id_as_int)


def _store_gguf_loaded_weight(param, loaded_weight, shard_id=None):
    loaded_weight = loaded_weight.detach().clone()
    if loaded_weight.dim() == 0:
        loaded_weight = loaded_weight.reshape(1)
    if shard_id is None:
        if isinstance(param, UninitializedParameter):
            param.materialize(tuple(loaded_weight.shape), device=param.device, dtype=loaded_weight.dtype)
        param.data.copy_(loaded_weight)
        return
    loaded_weight = loaded_weight.to(device=param.device)
    if shard_id not in param.shard_id_map:
        param.shard_id_map[shard_id] = len(param.data_container)
        param.data_container.append(loaded_weight)
        param.shard_id.append(shard_id)
    else:
        param.data_container[param.shard_id_map[shard_id]] = loaded_weight


def _store_gguf_weight_type(param, loaded_weight, shard_id=None):
    weight_type = int(torch.as_tensor(loaded_weight).reshape(-1)[0].item())
    if shard_id is None:
        param.weight_type = weight_type
        return
    param.shard_weight_type[shard_id] = weight_type
    if len(param.shard_weight_type) == 1:
        param.weight_type = weight_type


class GGUFWeightParameter(Parameter):
    def __new__(cls, data=None, **kwargs):
        p = super().__new__(cls, data, requires_grad=False)
        for k, v in kwargs.items():
            setattr(p, k, v)
        return p


class GGUFUninitializedParameter(UninitializedParameter):
    cls_to_become = Parameter


class GGUFUninitializedWeightParameter(GGUFUninitializedParameter):
    def _store(self, loaded_weight, shard_id=None):
        _store_gguf_loaded_weight(self, loaded_weight, shard_id)


class GGUFUninitializedWeightTypeParameter(GGUFUninitializedParameter):
    def _store(self, loaded_weight, shard_id=None):
        _store_gguf_weight_type(self, loaded_weight, shard_id)


def _resolve_gguf_weight_loader(layer, fallback_weight_loader=None):
    return getattr(layer, "weight_loader_v2", None) or fallback_weight_loader or _default_loader


def _resolve_gguf_weight_type_loader(layer, fallback_weight_loader=None):
    return _default_loader


def _default_loader(param, loaded_weight, loaded_shard_id=None):
    if isinstance(loaded_shard_id, tuple):
        for sid in loaded_shard_id:
            param._store(loaded_weight, shard_id=sid)
        return
    param._store(loaded_weight, shard_id=loaded_shard_id)


def _materialize_gguf_weight_parameter(layer, param_name):
    raw = getattr(layer, param_name)
    if isinstance(raw, GGUFWeightParameter):
        return
    data = (torch.empty(0, dtype=torch.uint8, device=raw.device)
            if isinstance(raw, UninitializedParameter) else raw.data)
    w = GGUFWeightParameter(data=data, weight_loader=raw.weight_loader, input_dim=raw.input_dim,
                            output_dim=raw.output_dim, tensor_shape=raw.tensor_shape)
    w.data_container = list(raw.data_container)
    w.shard_id = list(raw.shard_id)
    w.shard_id_map = dict(raw.shard_id_map)
    if len(w.data_container) == 1 and w.data.numel() == 0:
        w.data = w.data_container[0]
    raw.data_container.clear()
    raw.shard_id.clear()
    raw.shard_id_map.clear()
    layer.register_parameter(param_name, w)


def _materialize_gguf_weight_type_parameter(layer, param_name):
    raw = getattr(layer, param_name)
    if isinstance(raw, GGUFWeightParameter):
        return
    wt = GGUFWeightParameter(data=torch.empty(getattr(raw, "num_elements", 1), dtype=torch.uint8,
                                              device=raw.device),
                             weight_loader=raw.weight_loader)
    wt.weight_type = raw.weight_type
    wt.shard_weight_type = dict(raw.shard_weight_type)
    wt.num_elements = getattr(raw, "num_elements", 1)
    layer.register_parameter(param_name, wt)
