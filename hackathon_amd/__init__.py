"""MI355X-native one-step recurrent inference of the 4-tower ensemble
(xLSTM, Mamba2, RetNet, Hawk), behind the reference's process_batch() and
model APIs.

Layers
- `hackathon_amd.kernels`  the reference's fused state-step API on HIP kernels
- `hackathon_amd.engine`   the ensemble engine: HBM state store, packed
                           weights, layer-major tick (C++ / HIP library)
- `hackathon_amd.client`   NnInferenceClient.process_batch drop-in
"""

__all__ = ["kernels"]
