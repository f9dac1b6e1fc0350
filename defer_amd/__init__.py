"""MI355X-native (gfx950) per-token forward pass of defer.

``defer_amd.gpu`` binds the HIP library (include/defer_gpu.h);
``defer_amd.host`` binds the C++ host side (include/defer_host.h);
``defer_amd.synthetic`` builds the benchmark models and inputs.
"""
