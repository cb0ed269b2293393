"""loom_hip_hw_spec on the device: the reported properties agree with what
torch reads from the same device, the part is gfx950, and a workgroup may
use the LDS capacity the constraint scopes assume."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_device_section():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    spec = loom_hip.hw_spec(0)
    dev = spec["device"]
    props = torch.cuda.get_device_properties(0)
    print(f"hw_spec device: {dev}", flush=True)
    assert dev["compute_units"] == props.multi_processor_count
    assert dev["arch"].startswith("gfx950")
    assert dev["warp_size"] == spec["wave_size"] == 64
    assert dev["lds_bytes_per_workgroup"] >= spec["lds_bytes_per_workgroup"]
    assert dev["global_bytes"] == props.total_memory
