"""The few vLLM names the linear method uses. With vLLM installed they are vLLM's own; without
it (this image), minimal equivalents so the quant-method surface runs standalone: the linear
method base class, set_weight_attrs, and direct_register_custom_op (a torch.library op in the
"vllm" namespace with a fake implementation, as vLLM registers it)."""

import torch

try:
    from vllm.model_executor.layers.linear import LinearMethodBase, UnquantizedLinearMethod
    from vllm.model_executor.utils import set_weight_attrs
    from vllm.utils.torch_utils import direct_register_custom_op

    HAVE_VLLM = True
except ImportError:
    HAVE_VLLM = False

    class LinearMethodBase:
        """vLLM's LinearMethodBase interface: create_weights / apply / process_weights_after_loading."""

        def create_weights(self, layer, *args, **kwargs):
            raise NotImplementedError

        def apply(self, layer, x, bias=None):
            raise NotImplementedError

        def process_weights_after_loading(self, layer):
            return

    class UnquantizedLinearMethod(LinearMethodBase):
        def apply(self, layer, x, bias=None):
            return torch.nn.functional.linear(x, layer.weight, bias)

    def set_weight_attrs(weight, weight_attrs):
        for key, value in (weight_attrs or {}).items():
            setattr(weight, key, value)

    _vllm_lib = torch.library.Library("vllm", "FRAGMENT")

    def direct_register_custom_op(op_name, op_func, mutates_args=(), fake_impl=None, target_lib=None):
        schema = torch.library.infer_schema(op_func, mutates_args=mutates_args)
        lib = target_lib or _vllm_lib
        lib.define(op_name + schema)
        lib.impl(op_name, op_func, "CompositeExplicitAutograd")
        if fake_impl is not None:
            torch.library.register_fake(f"vllm::{op_name}", fake_impl, lib=lib)
