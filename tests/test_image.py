"""The DDR image container's region bookkeeping (hb_image with no device
memory, so no GPU) against the reference's own cases for DdrImage
(tools/compiler/ddr_image_test.cpp:14-92): aligned regions in order, reuse,
a name allocated again without reuse, Define, and the failure texts."""
from __future__ import annotations

import pytest

import hotarubi_amd as hb

CAP = 1 << 16
PAGE = hb.Image.PAGE


def image():
    return hb.Image(CAP, ctx=False)


def test_allocates_aligned_regions_in_order():
    im = image()
    assert im.alloc("a", 100) == 0
    assert im.alloc("b", 10) == PAGE
    assert im.alloc("c", 1, 16) == PAGE + 16
    assert im.end() == PAGE + 17
    regions = im.regions()
    assert len(regions) == 3 and regions[1][0] == "b"
    assert im.region("c") == (PAGE + 16, 1)


def test_reuse_returns_the_region_already_named():
    im = image()
    im.alloc("a", 100)
    im.set_reuse(True)
    assert im.alloc("a", 60) == 0
    assert im.end() == 100
    assert im.alloc("b", 8) == PAGE
    assert im.region("a") == (0, 100)
    assert len(im.regions()) == 2


def test_without_reuse_a_name_moves_to_a_new_region():
    im = image()
    im.alloc("a", 100)
    assert im.alloc("a", 200) == PAGE
    assert im.regions() == [("a", PAGE, 200)]


def test_define_names_a_range_inside_the_image():
    im = image()
    im.alloc("scratch", 2 * PAGE)
    im.define("part", PAGE, 100)
    assert [r[0] for r in im.regions()] == ["scratch", "part"]
    assert im.region("part") == (PAGE, 100)
    assert im.end() == 2 * PAGE


def expect_einval(fn, text):
    with pytest.raises(hb.HbError) as err:
        fn()
    assert err.value.code == hb.HB_EINVAL and text in err.value.message, err.value.message


def test_rejects_a_region_past_the_capacity():
    im = image()
    expect_einval(lambda: im.alloc("a", CAP + 1), "exceeds the image")


def test_rejects_reuse_with_more_bytes():
    im = image()
    im.alloc("a", 100)
    im.set_reuse(True)
    expect_einval(lambda: im.alloc("a", 101), "reused with 101 bytes")


def test_rejects_defining_past_the_end_or_a_taken_name():
    im = image()
    im.alloc("a", 100)
    expect_einval(lambda: im.define("b", 50, 51), "cannot define region b")
    expect_einval(lambda: im.define("a", 0, 10), "cannot define region a")


def test_rejects_an_unknown_name():
    expect_einval(lambda: image().region("a"), "no region named a")


def test_bytes_need_device_memory():
    im = image()
    im.alloc("a", 4)
    expect_einval(lambda: im.put(0, b"\x01"), "no device memory")
    expect_einval(lambda: im.put(CAP, b"\x01"), "exceed the image")
