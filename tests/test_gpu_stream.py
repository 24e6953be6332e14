"""Streaming-loop parity of the HIP path against the CPU oracle on the five configs."""
import pytest

import stream_check

pytestmark = pytest.mark.gpu


def test_c1_stream_prefix():
    tot = stream_check.run("c1", 40, check=set(range(40)), ring_check_every=5)
    assert tot["checked"] == 40 and tot["valid"] > 0


def test_c2_stream_prefix_co_occurrence():
    tot = stream_check.run("c2", 40, check=set(range(0, 40, 2)), ring_check_every=5)
    assert tot["valid"] > 0


def test_c3_warm_window():
    tot = stream_check.run("c3", 120, check={1, 60, 119}, ring_check_every=40)
    assert tot["valid"] > 0


def test_c4_warm_window():
    tot = stream_check.run("c4", 40, check={1, 39}, ring_check_every=20)
    assert tot["valid"] > 0


def test_c5_warm_window():
    tot = stream_check.run("c5", 24, check={1, 23}, ring_check_every=12)
    assert tot["valid"] > 0
