# SPDX-License-Identifier: Apache-2.0
"""GGUF linear method: the quant-method surface of the reference plugin
(plugin/vllm_gguf_plugin/quantization/linear.py), with its products served by this build's
gfx950 kernels through torch.ops._C_gguf.

Kept as the reference has it (same names, arguments and decisions):
  * _lcpp_op (linear.py:85-114): the op per (activation rows n, type, weight rows, K, packed);
  * _fused_mul_mat_gguf / _impl (:133-218): empty n, fp32-dst chunking of huge products
    (:117-130), x_q8 sharing, the >32-row packed and >8-row MMVQ splits;
  * _shard_weight / _shard_runs / _quantize_x_q8_1 (:221-268): one product per same-type run of
    a fused layer, one q8_1 quantisation shared by the runs that read it;
  * GGUFLinearMethod.create_weights / process_weights_after_loading / _pack_iq3 /
    _create_padded_weight_param / apply (:347-570).
What differs: the repack hook writes this build's IQ3_S tile layout (iq3_pack.py), and the
reference's stock CUDA / Triton dispatch for Route-L-off is not rebuilt (a quantized type with no
Route L op raises NotImplementedError).
"""

import os
from itertools import groupby

import torch

from .. import ops
from . import iq3_pack
from ._vllm import LinearMethodBase, UnquantizedLinearMethod, direct_register_custom_op, set_weight_attrs
from .params import (
    GGUFUninitializedWeightParameter,
    GGUFUninitializedWeightTypeParameter,
    GGUFWeightParameter,
    _gguf_ordered_shard_ids,
    _materialize_gguf_weight_parameter,
    _materialize_gguf_weight_type_parameter,
    _resolve_gguf_weight_loader,
    _resolve_gguf_weight_type_loader,
)
from .utils import DEQUANT_TYPES, UNQUANTIZED_TYPES, WeightType

_IQ3_TYPES = (WeightType.IQ3_S, WeightType.IQ3_XXS)
# The packed IQ3_XXS GEMV stages one activation row's q8_1 (36 bytes per 32 values) in at most
# 96 KB of LDS: K <= 87040 (K % 512 == 0).
_XXS_PACK_MAX_K = 87040
# fewest activation rows at which lcpp_mul_mat_vec_own is routed (up to 8)
_OWN_MIN_ROWS = {WeightType.Q4_K: 3, WeightType.IQ2_S: 1}
# most activation rows at which IQ1_M is routed to MMVQ (in 8-row calls above 8)
_IQ1_M_MAX_ROWS = 32
_MMA_K_TYPES = (WeightType.Q4_K, WeightType.IQ4_XS, WeightType.IQ2_S)
# packed IQ3: the decode op up to here, the tiled op above
PACKED_VEC_MAX_ROWS = 8
# ops that quantize X themselves (MMQ block layout); the others read apply()'s shared x_q8
_OWN_QUANTIZE_OPS = ("lcpp_mul_mat_q", "lcpp_mul_mat_mma_k", "lcpp_mul_mat_iq3_packed")
# ops that write X's dtype directly (here every op does; kept for the chunking rule below)
_X_DTYPE_OPS = ("lcpp_mul_mat_mma_k", "lcpp_mul_mat_iq3_packed", "lcpp_mul_mat_vec_iq3")
# most fp32 dst bytes one call may allocate before row-chunking (vocab-sized heads)
_FP32_DST_BUDGET = 256 << 20

# kill switches (default on), each excluding one path, as the reference's
_MMA_K_ON = os.environ.get("VLLM_GGUF_MMA_K", "1") != "0"
_IQ3_TILED_ON = os.environ.get("VLLM_GGUF_IQ3_TILED", "1") != "0"
_IQ1M_MMVQ_ON = os.environ.get("VLLM_GGUF_IQ1M_MMVQ", "1") != "0"
# debug: every eager product on a vocab-sized weight (> 50,000 rows) at > 8 activation rows is
# recomputed with the decode op in 8-row calls and the per-row disagreement appended as one JSON
# line to this file (synchronises: debug only; reference linear.py:67-70,143-163)
_HEADCHECK = os.environ.get("VLLM_GGUF_HEADCHECK")


def _mma_k_wins(weight_type: int, n: int, rows: int, k: int) -> bool:
    """9..32 activation rows on weights above 2048 rows; IQ4_XS at 17..32 rows only from
    rows*K >= 12288*5120 (reference linear.py:75-82)."""
    if weight_type not in _MMA_K_TYPES or not 9 <= n <= 32 or rows <= 2048 or not _MMA_K_ON:
        return False
    return n <= 16 or weight_type != WeightType.IQ4_XS or rows * k >= 12288 * 5120


def _lcpp_op(n: int, weight_type: int, rows: int, k: int, packed: bool = False) -> str | None:
    """The Route L op name for n activation rows times a weight_type weight of `rows` rows and k
    columns, or None if there is none; packed: the layer's IQ3 runs are in the tile layout."""
    if packed and weight_type in _IQ3_TYPES:
        if n <= PACKED_VEC_MAX_ROWS or not _IQ3_TILED_ON:
            return "lcpp_mul_mat_vec_iq3_mma_packed"
        return "lcpp_mul_mat_iq3_packed"
    if weight_type == WeightType.IQ1_M:
        return "lcpp_mul_mat_vec_q" if n <= _IQ1_M_MAX_ROWS and (n <= 8 or _IQ1M_MMVQ_ON) else None
    if n <= 8 and weight_type in _IQ3_TYPES:
        return "lcpp_mul_mat_vec_iq3_mma" if n >= 6 else "lcpp_mul_mat_vec_iq3"
    if _OWN_MIN_ROWS.get(weight_type, 9) <= n <= 8 and rows > 2048:
        return "lcpp_mul_mat_vec_own"
    if _mma_k_wins(weight_type, n, rows, k):
        return "lcpp_mul_mat_mma_k"
    return "lcpp_mul_mat_vec_q" if n < 8 else "lcpp_mul_mat_q"


def _fused_mul_mat_gguf_chunked(x: torch.Tensor, weight: torch.Tensor, weight_type: int,
                                packed: bool) -> torch.Tensor:
    """_fused_mul_mat_gguf in activation-row chunks whose fp32 dst fits _FP32_DST_BUDGET
    (multiples of 128 rows), into one X-dtype output; each chunk routes and quantizes itself."""
    n, rows = x.shape[0], weight.shape[0]
    step = max(1, _FP32_DST_BUDGET // (rows * 4))
    if step >= 128:
        step -= step % 128
    out = torch.empty(n, rows, dtype=x.dtype, device=x.device)
    for i in range(0, n, step):
        out[i:i + step] = _fused_mul_mat_gguf(x[i:i + step], weight, weight_type, None, packed)
    return out


def _fused_mul_mat_gguf(x: torch.Tensor, weight: torch.Tensor, weight_type: int,
                        x_q8: torch.Tensor | None = None, packed: bool = False) -> torch.Tensor:
    """x @ weight.T. x_q8: x already quantized by _quantize_x_q8_1 for this product and others
    on the same x; used if this product's op reads q8_1."""
    y = _fused_mul_mat_gguf_impl(x, weight, weight_type, x_q8, packed)
    if (_HEADCHECK and weight.shape[0] > 50000 and x.shape[0] > 8 and weight_type in ops.LCPP_QUANT_TYPES
            and not packed and not torch.cuda.is_current_stream_capturing()):
        _headcheck(x, weight, weight_type, y, _lcpp_op(x.shape[0], weight_type, weight.shape[0], x.shape[1], packed))
    return y


def _headcheck(x, weight, weight_type, y, name):
    """The VLLM_GGUF_HEADCHECK record of one product: the decode op (lcpp_mul_mat_vec_q in 8-row
    calls) beside the routed op's y; per activation row the largest difference relative to the row's
    largest value, the rows above 5 %, the rows whose argmax differs, and whether x and y are
    finite (reference linear.py:146-163)."""
    import json

    alt = torch.cat([torch.ops._C_gguf.lcpp_mul_mat_vec_q(weight, x[i:i + 8], weight_type, weight.shape[0])
                     for i in range(0, x.shape[0], 8)]).float()
    yf = y.float()
    rel = ((yf - alt).abs().amax(-1) / alt.abs().amax(-1).clamp_min(1e-6)).nan_to_num(1e9)
    rec = {"n": x.shape[0], "rows": weight.shape[0], "route": name, "max_rel": float(rel.max()),
           "bad_rows": (rel > 0.05).nonzero().flatten().tolist(),
           "argmax_diff_rows": (yf.argmax(-1) != alt.argmax(-1)).nonzero().flatten().tolist(),
           "x_finite": bool(torch.isfinite(x).all()), "y_finite": bool(torch.isfinite(y).all()),
           "x_absmax": float(x.float().abs().max())}
    with open(_HEADCHECK, "a") as f:
        f.write(json.dumps(rec) + "\n")


def _fused_mul_mat_gguf_impl(x: torch.Tensor, weight: torch.Tensor, weight_type: int,
                             x_q8: torch.Tensor | None = None, packed: bool = False) -> torch.Tensor:
    if x.shape[0] == 0:
        return torch.empty(x.shape[0], weight.shape[0], dtype=x.dtype, device=x.device)
    if weight_type in UNQUANTIZED_TYPES:
        return x @ weight.T
    name = None
    if ops.LCPP_ENABLED and weight_type in ops.LCPP_QUANT_TYPES:
        name = _lcpp_op(x.shape[0], weight_type, weight.shape[0], x.shape[1], packed)
    if name is None:
        raise NotImplementedError(f"Unsupported GGUF quantization type: {WeightType(weight_type)!r} "
                                  f"(no Route L op for {x.shape[0]} rows in this build)")
    n, rows = x.shape[0], weight.shape[0]
    if name not in _X_DTYPE_OPS and x.dtype != torch.float32 and n * rows * 4 > _FP32_DST_BUDGET:
        return _fused_mul_mat_gguf_chunked(x, weight, weight_type, packed)
    op = getattr(torch.ops._C_gguf, name)
    if name in _OWN_QUANTIZE_OPS:
        return op(weight, x, weight_type, rows)
    if name == "lcpp_mul_mat_vec_iq3_mma_packed" and n > 32:  # VLLM_GGUF_IQ3_TILED=0
        b = x.shape[1] // 32 * 36
        return torch.cat([op(weight, x[i:i + 32], weight_type, rows,
                             None if x_q8 is None else x_q8[i * b:(i + 32) * b])
                          for i in range(0, n, 32)])
    if name == "lcpp_mul_mat_vec_q" and n > 8:  # IQ1_M: at most 8 rows per call
        b = x.shape[1] // 32 * 36
        return torch.cat([op(weight, x[i:i + 8], weight_type, rows,
                             None if x_q8 is None else x_q8[i * b:(i + 8) * b])
                          for i in range(0, n, 8)])
    return op(weight, x, weight_type, rows, x_q8)


def _shard_weight(weight: torch.Tensor, start: int, end: int, size: int) -> torch.Tensor:
    """Rows start:end, first `size` bytes, of a padded multi-shard weight: with Route L each
    same-type run is stored contiguously from its first shard's row, so a run is a view."""
    if ops.LCPP_ENABLED:
        rows = end - start
        return weight[start:end].view(-1)[:rows * size].view(rows, size)
    return weight[start:end, :size].contiguous()


def _shard_runs(weight: torch.Tensor, shard_ids: list, weight_types: list):
    """(weight view, type) per run of adjacent same-type shards of a padded multi-shard weight."""
    offsets = weight.shard_offset_map
    key = (lambda p: p[1]) if ops.LCPP_ENABLED else (lambda p: p[0])
    for _, run in groupby(zip(shard_ids, weight_types), key=key):
        ids, types = zip(*run)
        start, _, size = offsets[ids[0]]
        yield _shard_weight(weight, start, offsets[ids[-1]][1], size), types[0]


def _q8_1_type(n: int, k: int, weight_types: list[int], weight_rows: list[int], packed: bool = False):
    """The type the shared q8_1 of an [n, k] x is quantized for: the first run whose op reads
    q8_1 (reference linear.py:251-268), or None when no run's op does (or n == 0)."""
    q8_1 = [t for t, rows in zip(weight_types, weight_rows)
            if t in ops.LCPP_QUANT_TYPES and _lcpp_op(n, t, rows, k, packed) not in (None, *_OWN_QUANTIZE_OPS)]
    return q8_1[0] if n and q8_1 else None


def _quantize_x_q8_1(x: torch.Tensor, weight_types: list[int], weight_rows: list[int],
                     packed: bool = False) -> torch.Tensor:
    """x as q8_1 blocks, quantized once for every product on x whose op reads q8_1 (with the
    first such run's type); an unfilled buffer of the same size when none does."""
    qt = _q8_1_type(x.shape[0], x.shape[1], weight_types, weight_rows, packed)
    if qt is not None:
        return torch.ops._C_gguf.lcpp_quantize_q8_1(x, qt, False, False)
    return _quantize_x_q8_1_fake(x, weight_types, weight_rows)


def _fused_mul_mat_gguf_fake(x: torch.Tensor, weight: torch.Tensor, weight_type: int,
                             x_q8: torch.Tensor | None = None, packed: bool = False) -> torch.Tensor:
    return torch.empty(x.shape[0], weight.shape[0], dtype=x.dtype, device=x.device)


def _quantize_x_q8_1_fake(x: torch.Tensor, weight_types: list[int], weight_rows: list[int],
                          packed: bool = False) -> torch.Tensor:
    return torch.empty(x.shape[0] * x.shape[1] // 32 * 36, dtype=torch.uint8, device=x.device)


_DENSE_MAX_ROWS = 128  # the small-weight route's limits (reference linear.py:281-291)
_DENSE_MAX_N = 8


def _dense_ok(x: torch.Tensor, weight: torch.Tensor, bias) -> bool:
    """The layouts torch.ops._C_gguf.dense_mul_mat takes: one float dtype, unit inner strides,
    K % 32 == 0, data and row strides 16-byte aligned."""
    if bias is not None or not x.is_cuda or x.dim() != 2 or weight.dim() != 2 or x.dtype != weight.dtype:
        return False
    if x.shape[0] > _DENSE_MAX_N or weight.shape[0] > _DENSE_MAX_ROWS or x.shape[1] % 32:
        return False
    es = x.element_size()
    return (x.stride(1) == 1 and weight.stride(1) == 1 and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0
            and (x.shape[0] <= 1 or (x.stride(0) * es) % 16 == 0)
            and (weight.shape[0] <= 1 or (weight.stride(0) * es) % 16 == 0))


def _unquantized_gemm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """x @ weight.T (+ bias) for a GGUF F32/F16/BF16 tensor (reference linear.py:281-291). A weight
    of at most 128 rows times up to 8 activation rows runs the library's small dense GEMV (the
    reference batches a GEMV there: a library GEMM picks a few tiny workgroups for that shape);
    everything else is torch's linear."""
    if _dense_ok(x, weight, bias):
        return torch.ops._C_gguf.dense_mul_mat(weight, x)
    return torch.nn.functional.linear(x, weight, bias)


def _unquantized_gemm_fake(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    return x.new_empty(x.shape[0], weight.shape[0])


def _register_custom_ops():
    if hasattr(torch.ops.vllm, "_fused_mul_mat_gguf"):
        return
    direct_register_custom_op(op_name="_fused_mul_mat_gguf", op_func=_fused_mul_mat_gguf,
                              fake_impl=_fused_mul_mat_gguf_fake)
    direct_register_custom_op(op_name="_quantize_x_q8_1", op_func=_quantize_x_q8_1,
                              fake_impl=_quantize_x_q8_1_fake)
    direct_register_custom_op(op_name="_gguf_unquantized_gemm", op_func=_unquantized_gemm,
                              fake_impl=_unquantized_gemm_fake)


_register_custom_ops()
fused_mul_mat_gguf = torch.ops.vllm._fused_mul_mat_gguf
quantize_x_q8_1 = torch.ops.vllm._quantize_x_q8_1
unquantized_gemm = torch.ops.vllm._gguf_unquantized_gemm


class GGUFUnquantizedLinearMethod(UnquantizedLinearMethod):
    """The GGUF's F32/F16/BF16 tensors, product in a custom op."""

    def apply(self, layer, x, bias=None):
        if x.dim() != 2:
            return super().apply(layer, x, bias)
        return unquantized_gemm(x, layer.weight, bias)


class GGUFLinearMethod(LinearMethodBase):
    """Linear method for GGUF."""

    # apply() sends IQ3 weights to the packed ops (_pack_iq3)
    pack_iq3 = True

    def __init__(self, quant_config=None, layout=None) -> None:
        self.quant_config = quant_config
        self.layout = layout

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: list[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs):
        del output_size
        self.params_dtype = params_dtype
        output_size_per_partition = sum(output_partition_sizes)
        fallback_weight_loader = extra_weight_attrs.pop("weight_loader", None)
        weight_loader = _resolve_gguf_weight_loader(layer, fallback_weight_loader)

        weight = GGUFUninitializedWeightParameter(requires_grad=False)
        set_weight_attrs(weight, {
            "weight_loader": weight_loader,
            "input_dim": 1,
            "output_dim": 0,
            "tensor_shape": (output_size_per_partition, input_size_per_partition),
            "data_container": [],
            "shard_id": [],
            "shard_id_map": {},
        })
        set_weight_attrs(weight, extra_weight_attrs)
        layer.register_parameter("weight", weight)

        weight_type = GGUFUninitializedWeightTypeParameter(requires_grad=False)
        set_weight_attrs(weight_type, {
            "weight_loader": _resolve_gguf_weight_type_loader(layer, fallback_weight_loader),
            "weight_type": 0,
            "shard_weight_type": {},
            "num_elements": len(output_partition_sizes),
            "ignore_warning": True,
        })
        set_weight_attrs(weight_type, extra_weight_attrs)
        layer.register_parameter("weight_type", weight_type)

    def process_weights_after_loading(self, layer: torch.nn.Module):
        _materialize_gguf_weight_parameter(layer, "weight")
        _materialize_gguf_weight_type_parameter(layer, "weight_type")
        weight_type = layer.weight_type.weight_type
        if not (weight_type in UNQUANTIZED_TYPES or weight_type in DEQUANT_TYPES):
            raise ValueError(f"Unsupported GGUF quantization type {WeightType(weight_type)!r} in layer {layer}.")
        self._create_padded_weight_param(layer)
        if ops.LCPP_ENABLED and self.pack_iq3:
            self._pack_iq3(layer)

    def _pack_iq3(self, layer: torch.nn.Module) -> None:
        """Store the layer's IQ3_S / IQ3_XXS runs in iq3_pack's layout, in place, and set
        weight.iq3_packed (reference linear.py:437-457); apply() then routes them to the packed
        ops. All or nothing per layer: every IQ3 run must have a multiple of 16 rows and 16-byte
        aligned bytes, and be on the GPU (the repack runs there); an IQ3_XXS run's K must fit the
        packed GEMV's X staging (_XXS_PACK_MAX_K)."""
        weight = layer.weight
        if getattr(weight, "iq3_packed", False):
            return
        if hasattr(weight, "shard_offset_map"):
            types = layer.weight_type.shard_weight_type
            fallback = layer.weight_type.weight_type
            runs = list(_shard_runs(weight, weight.shard_id, [types.get(i, fallback) for i in weight.shard_id]))
        else:
            runs = [(weight.data, layer.weight_type.weight_type)]
        runs = [(w, t) for w, t in runs if t in _IQ3_TYPES]
        if not runs or any(w.shape[0] % iq3_pack.ROWS or w.data_ptr() % 16 or not w.is_cuda for w, _ in runs):
            return
        if any(t == WeightType.IQ3_XXS and w.shape[1] // 98 * 256 > _XXS_PACK_MAX_K for w, t in runs):
            return
        for w, t in runs:
            iq3_pack.pack_(w, t)
        weight.iq3_packed = True

    def _create_padded_weight_param(self, layer: torch.nn.Module):
        """One zero-padded [sum rows, max row bytes] uint8 buffer for a multi-shard weight; with
        Route L each run of adjacent same-type shards is stored contiguously (see _shard_weight)."""
        weight = layer.weight
        data_container = weight.data_container
        if len(data_container) <= 1:
            return
        dtype = {d.dtype for d in data_container}
        assert len(dtype) == 1, f"Data container has mixed dtypes: {dtype}"
        padded_side = max(d.size(1) for d in data_container)
        concat_side = sum(d.size(0) for d in data_container)
        padded = torch.zeros((concat_side, padded_side), dtype=next(iter(dtype)), device=data_container[0].device)
        offsets = {}
        ordered = _gguf_ordered_shard_ids(weight.shard_id)
        types = layer.weight_type.shard_weight_type
        cur = run_start = 0
        run_type = None
        for idx in ordered:
            d = data_container[weight.shard_id_map[idx]]
            start, end, size = cur, cur + d.size(0), d.size(1)
            if ops.LCPP_ENABLED:
                wtype = types.get(idx, layer.weight_type.weight_type)
                if wtype != run_type:
                    run_start, run_type = start, wtype
                at = run_start * padded_side + (start - run_start) * size
                padded.view(-1)[at:at + (end - start) * size] = d.reshape(-1)
            else:
                padded[start:end, :size] = d
            offsets[idx] = (start, end, size)
            cur = end
        p = GGUFWeightParameter(data=padded, weight_loader=weight.weight_loader, input_dim=weight.input_dim,
                                output_dim=weight.output_dim, tensor_shape=weight.tensor_shape)
        p.data_container = []
        p.shard_id = ordered
        p.shard_id_map = dict(weight.shard_id_map)
        set_weight_attrs(p, {"shard_offset_map": offsets})
        weight.data_container.clear()
        layer.register_parameter("weight", p)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        if self.layout is not None:
            x = self.layout.input_to_gguf(x)
        shard_id = layer.weight.shard_id
        packed = getattr(layer.weight, "iq3_packed", False)
        if shard_id:
            shard_id = ["q", "k", "v"] if "q" in shard_id else shard_id
            weight = layer.weight
            fallback = layer.weight_type.weight_type
            shard_types = [layer.weight_type.shard_weight_type.get(i, fallback) for i in shard_id]
            if len(set(shard_types)) == 1:
                out = fused_mul_mat_gguf(x, weight, shard_types[0], None, packed)
                if bias is not None:
                    out.add_(bias)
                return out
            runs = list(_shard_runs(weight, shard_id, shard_types))
            x_q8 = (quantize_x_q8_1(x, [t for _, t in runs], [w.shape[0] for w, _ in runs], packed)
                    if ops.LCPP_ENABLED else None)
            out = torch.cat([fused_mul_mat_gguf(x, w, t, x_q8, packed) for w, t in runs], dim=1)
        else:
            out = fused_mul_mat_gguf(x, layer.weight, layer.weight_type.weight_type, None, packed)
        if bias is not None:
            out.add_(bias)
        return out
