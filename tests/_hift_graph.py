"""The reference's graph builders as node lists (HiFT and the CFM decoder's
causal block): the package's NodeList, under the name the tests use."""
from chatterbox_amdvulkan_amd.ggml_nodes import NodeList as HiftGraph  # noqa: F401
