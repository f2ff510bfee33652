"""MI355X (gfx950) decode path of GPULlama3.java behind the C ABI of include/gl3.h.

Import with the package directory `gpullama3.java_amd/` on sys.path:
    sys.path.insert(0, "<repo>/gpullama3.java_amd"); import gpullama3_hip
"""
from . import _lib
from .model import CONFIGS, ModelShape, TensorSpec, gl3_config, synth_model, tensor_specs
from .plan import HipMasterPlan, device_name

__all__ = ["CONFIGS", "ModelShape", "TensorSpec", "gl3_config", "synth_model", "tensor_specs",
           "HipMasterPlan", "device_name", "_lib"]
