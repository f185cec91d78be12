"""The observability helpers and the e2e configuration, on the CPU."""

import time

from flash_lab.observe import FIELDS, ClockSampler, roctx_range


def test_clock_sampler_windows():
    with ClockSampler(interval_ms=10) as clocks:
        start = time.time()
        time.sleep(0.05)
        end = time.time()
    window = clocks.window(start, end)
    if not clocks.available:  # no GPU visible to amdsmi (the CPU test machine)
        assert window is None and clocks.samples == []
        return
    assert window["samples"] >= 1
    assert set(window) - {"samples"} <= set(FIELDS)


def test_clock_sampler_window_statistics():
    clocks = ClockSampler()
    clocks.samples = [(1.0, (2100.0, 1900.0, 900.0, 60.0)), (2.0, (1700.0, 1900.0, None, 70.0))]
    window = clocks.window(0.5, 2.5)
    assert window["samples"] == 2
    assert window["gfx_mhz"] == {"min": 1700.0, "median": 1900.0, "max": 2100.0}
    assert window["power_w"] == {"min": 900.0, "median": 900.0, "max": 900.0}
    # A window between samples gets the nearest one.
    assert clocks.window(1.1, 1.2)["temp_c"]["median"] == 60.0


def test_roctx_range_nests():
    with roctx_range("outer"):
        with roctx_range("inner"):
            pass


def test_e2e_config_is_llama_31_8b_shaped():
    import e2e

    c = e2e.llama_config(32)
    assert (c.num_hidden_layers, c.hidden_size, c.intermediate_size) == (32, 4096, 14336)
    assert (c.num_attention_heads, c.num_key_value_heads, c.head_dim) == (32, 8, 128)
    assert c.vocab_size == 128256
    assert c.rope_parameters["rope_theta"] == 500000.0
