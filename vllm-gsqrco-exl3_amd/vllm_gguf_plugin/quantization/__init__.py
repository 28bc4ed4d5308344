"""The GGUF quant method of the plugin (linear method, routing, repack hook)."""
