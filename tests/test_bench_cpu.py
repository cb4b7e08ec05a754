"""CPU checks of bench.py helpers that need no GPU: the parser of the board
power/clock samples behind `bench.py --profile <K> --power S`."""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _metric(watts, clocks):
    """The shape `amd-smi metric -g 0 -p -c --json` prints (one GPU, 8 XCD
    clocks plus memory and media clocks that must be ignored)."""
    clock = {f"gfx_{i}": {"clk": {"value": c, "unit": "MHz"},
                          "min_clk": {"value": 500, "unit": "MHz"},
                          "max_clk": {"value": 2400, "unit": "MHz"},
                          "clk_locked": "DISABLED", "deep_sleep": "ENABLED"}
             for i, c in enumerate(clocks)}
    clock["mem_0"] = {"clk": {"value": 2000, "unit": "MHz"}}
    clock["fclk_0"] = {"clk": {"value": 1800, "unit": "MHz"}}
    return json.dumps({"gpu_data": [{"gpu": 0,
                                     "power": {"socket_power": {"value": watts, "unit": "W"},
                                               "gfx_voltage": "N/A"},
                                     "clock": clock}]})


def test_parse_takes_socket_power_and_median_gfx_clock():
    w, mhz = bench.parse_amdsmi_metric(_metric(1386, [2130, 2139, 2140, 2135, 2139, 2150, 2100, 2139]))
    assert w == 1386.0
    assert mhz == 2139.0      # median of the 8 XCDs; mem/fclk not counted


def test_parse_rejects_output_without_the_fields():
    assert bench.parse_amdsmi_metric("") is None
    assert bench.parse_amdsmi_metric("not json") is None
    assert bench.parse_amdsmi_metric(json.dumps({"gpu_data": []})) is None
    no_gfx = json.loads(_metric(900, []))
    assert bench.parse_amdsmi_metric(json.dumps(no_gfx)) is None
    na = json.loads(_metric(900, [2000]))
    na["gpu_data"][0]["power"]["socket_power"]["value"] = "N/A"
    assert bench.parse_amdsmi_metric(json.dumps(na)) is None
