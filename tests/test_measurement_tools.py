"""The measurement harness's trace and counter arithmetic, on synthetic
rocprofv3 rows (no GPU): how a dispatch is classified by what ran before it,
and how counter bytes are scaled by the plain copy of known size."""

from __future__ import annotations

import pytest

from mlc.bench.summarize import COPY_BYTES, _counter_bytes, _loop_us
from mlc.bench.trace_split import classify, report


def _row(name, start, end):
    return {"Kernel_Name": name, "Start_Timestamp": str(start), "End_Timestamp": str(end)}


def test_dispatches_are_classified_by_their_predecessor():
    fill = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<unsigned char>>"
    gemm = "Cijk_Alik_Bljk_HHS_BH_MT96x128x64"
    rows = [
        _row(gemm, 0, 10_000),
        _row("mlc_a", 11_000, 16_000),        # after a GEMM: in sequence, 5 us
        _row("mlc_a", 17_000, 20_000),        # after itself: loop, 3 us
        _row("mlc_a", 21_000, 24_000),        # loop, 3 us
        _row(fill, 25_000, 225_000),
        _row("mlc_a", 226_000, 233_000),      # after the fill, 7 us
        _row("mlc_b", 234_000, 236_000),      # after another generated kernel: in sequence
    ]
    # out of order on input: classification follows start time
    split = classify(list(reversed(rows)))
    assert split["mlc_a"] == {"in sequence": [5.0], "loop": [3.0, 3.0], "after fill": [7.0]}
    assert split["mlc_b"] == {"in sequence": [2.0]}
    table = report(split, {"mlc_a": 24_000_000})
    # 24 MB in 3 us is 8 TB/s: the loop column reads 1.000 of peak
    assert "| `mlc_a` | 2, 3.00 | 1, 7.00 | 1, 5.00 | 1.000 | 0.429 | 0.600 |" in table
    # classes that never occur are left out of the table
    assert "after fill" not in report({"mlc_c": {"loop": [1.0]}})


def test_loop_durations_take_only_back_to_back_dispatches():
    rows = [_row("k", 0, 4000), _row("k", 5000, 8000), _row("j", 9000, 10_000),
            _row("k", 11_000, 15_000)]
    assert dict(_loop_us(rows)) == {"k": [3.0]}


def test_counter_bytes_are_scaled_by_the_plain_copy():
    # the copy's true traffic is 1 GiB; a counter reading half of it in KiB
    # gives a scale of 2, applied to every kernel's reading
    half = COPY_BYTES / 2 / 1024
    rows = [{"Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Value": str(half)},
            {"Kernel_Name": "mlc_x(args)", "Counter_Value": "100"},
            {"Kernel_Name": "mlc_x", "Counter_Value": "300"}]
    scale, per = _counter_bytes(rows)
    assert scale == pytest.approx(2.0)
    assert per["mlc_x"] == [100.0, 300.0]


def test_counter_bytes_need_the_copy():
    with pytest.raises(SystemExit, match="1 GiB copy"):
        _counter_bytes([{"Kernel_Name": "mlc_x", "Counter_Value": "1"}])


def test_producer_split_groups_by_the_kernel_that_wrote_the_input(tmp_path):
    import csv

    from mlc.bench.producer import split

    gemm = "Cijk_Alik_Bljk_HHS_BH_MT64x64x32"
    copy = "void at::native::elementwise_kernel<128, 4, direct_copy_kernel_cuda>"
    rows = [_row(gemm, 0, 10_000), _row("mlc_s", 12_000, 19_000),     # after bmm: 7 us, gap 2
            _row(copy, 20_000, 23_000), _row("mlc_s", 24_000, 30_000),  # after copy: 6 us, gap 1
            _row("mlc_s", 31_000, 36_000)]                              # after itself: 5 us
    with open(tmp_path / "t_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    text = split(str(tmp_path), None)
    assert text.startswith("`mlc_s`")
    assert "| after the library bmm | 1 | 7.00 | 7.00 | 2.00 |" in text
    assert "| after a torch copy | 1 | 6.00 | 6.00 | 1.00 |" in text
    assert "| after itself | 1 | 5.00 | 5.00 | 1.00 |" in text
