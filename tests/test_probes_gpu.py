"""The device-figure probes bench.py reports beside the roofline fractions (vkllm_hip_probe_stream_read,
vkllm_hip_probe_launch_gap; no counterpart in the reference): plausible values on an MI355X, refused arguments."""
import pytest

pytestmark = pytest.mark.gpu


def test_stream_read_rate(ctx):
    med, best = ctx.probe_stream_read(64 << 20, 4)
    print(f"[probe] stream read of 64 MiB windows: median {med:.0f} GB/s, best {best:.0f} GB/s", flush=True)
    # below the 8 TB/s of HBM3E (no window is in the memory-side cache), and far above a host copy
    assert 1000.0 < med <= best < 8000.0


def test_launch_gap(ctx):
    us = ctx.probe_launch_gap(64, 1)
    print(f"[probe] dependent empty launch: {us:.2f} us", flush=True)
    assert 0.05 < us < 50.0


def test_refused_arguments(ctx, vk):
    for window, reps in ((33 << 20, 4), (0, 4), (2 << 30, 4), (64 << 20, 0)):
        with pytest.raises(vk.VkllmError) as e:
            ctx.probe_stream_read(window, reps)
        assert e.value.code == vk.ERR_ARGS
    for launches, blocks in ((0, 1), (5000, 1), (8, 0)):
        with pytest.raises(vk.VkllmError) as e:
            ctx.probe_launch_gap(launches, blocks)
        assert e.value.code == vk.ERR_ARGS
