"""MI355X (gfx950) AWQ W4A16 linear engine for SGLite.

* ``sglite_amd.quantization`` -- drop-in for SGLite's quantization-method API
  (AWQConfig / AWQLinearMethod, AWQMarlinConfig / AWQMarlinLinearMethod).
* ``sglite_amd.ops`` -- torch-facing wrappers of the C ABI (libsglite_awq.so,
  declared in include/sglite_awq.h).
* ``sglite_amd.linear`` -- the tensor-parallel linear plumbing that drives a
  linear method through create/load/process/apply.
* ``sglite_amd.model_config`` -- AWQ quantization-config detection.
"""

__version__ = "0.1.0"
