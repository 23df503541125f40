"""Checkpoint input and output (Kandle's packages/core/src/io): safetensors files and sharded indexes."""
from .safetensors import (SafetensorFile, SafetensorGroup, SafetensorLayer, host_array, load_safetensor,
                          parse_header_size, parse_safetensor_file, parse_sharded_index, save_safetensors,
                          tensor_from_safetensor_layer)

__all__ = ["SafetensorFile", "SafetensorGroup", "SafetensorLayer", "host_array", "load_safetensor",
           "parse_header_size", "parse_safetensor_file", "parse_sharded_index", "save_safetensors",
           "tensor_from_safetensor_layer"]
