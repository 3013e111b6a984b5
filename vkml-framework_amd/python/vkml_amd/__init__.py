"""Python side of vkml-mi355x: ctypes bindings to the C ABIs (include/vkml_hip.h,
include/vkml_llama.h) plus the synthetic-model tools. The bindings load the
in-tree libvkml_hip.so / libvkml.so and raise if they are missing."""
from . import gguf, synth  # noqa: F401
