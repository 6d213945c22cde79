"""bench.py's HBM-traffic measurement: parsing of rocprofv3 counter files
(the counter passes themselves need a GPU; the driver's bench run makes
them)."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = ("Correlation_Id,Dispatch_Id,Agent_Id,Queue_Id,Process_Id,Thread_Id,Grid_Size,"
          "Kernel_Id,Kernel_Name,Workgroup_Size,LDS_Block_Size,Scratch_Size,VGPR_Count,"
          "Accum_VGPR_Count,SGPR_Count,Counter_Name,Counter_Value,Start_Timestamp,"
          "End_Timestamp")


def bench():
    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def row(dispatch, kernel, counter, value):
    return (f'{dispatch},{dispatch},1,1,1,1,131072,{dispatch},"{kernel}",512,0,0,0,0,0,'
            f'{counter},{value},0,1')


def test_parse_counter_csv(tmp_path):
    b = bench()
    k = "void nut::(anonymous namespace)::token_kernel<Geo<1, 2048>, true, false>(nut::TokenArgs)"
    lines = [HEADER,
             row(1, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 12.0),  # upload copy
             row(2, k, "FETCH_SIZE", 4000.0), row(2, k, "FETCH_SIZE", 500.0),  # two XCD rows
             row(3, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 524288.0),
             row(4, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 524290.0),
             row(5, "qkv_fast_kernel<1, 2>", "FETCH_SIZE", 99.0),
             row(6, k, "WRITE_SIZE", 7.0)]
    f = tmp_path / "run_counter_collection.csv"
    f.write_text("\n".join(lines) + "\n")
    kernel, copy = b.parse_counter_csv([str(f)], "FETCH_SIZE")
    assert kernel == pytest.approx(4500.0)  # rows of one dispatch summed
    assert copy == pytest.approx(524290.0)  # the largest copy dispatch


def test_parse_counter_csv_missing(tmp_path):
    b = bench()
    f = tmp_path / "run_counter_collection.csv"
    f.write_text(HEADER + "\n" + row(1, "qkv_fast_kernel<1, 2>", "FETCH_SIZE", 1.0) + "\n")
    with pytest.raises(RuntimeError):
        b.parse_counter_csv([str(f)], "FETCH_SIZE")


def test_parse_counter_csv_wide_kernel(tmp_path):
    """The 7B-width decode runs on wide_kernel: its dispatches count as the
    decode launches, prefill kernels do not."""
    b = bench()
    k = "void nut::(anonymous namespace)::wide_kernel<WideGeo<1>, true>(nut::TokenArgs)"
    lines = [HEADER,
             row(1, "prefill_gemm_kernel<1>", "WRITE_SIZE", 900.0),
             row(2, k, "WRITE_SIZE", 30.0), row(2, k, "WRITE_SIZE", 2.0),
             row(3, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 1048576.0)]
    f = tmp_path / "run_counter_collection.csv"
    f.write_text("\n".join(lines) + "\n")
    kernel, copy = b.parse_counter_csv([str(f)], "WRITE_SIZE")
    assert kernel == pytest.approx(32.0)
    assert copy == pytest.approx(1048576.0)


def test_add_traffic_ratio():
    b = bench()
    line = {"roofline": {"bytes_per_launch": 1000, "traffic": None},
            "screened_roofline": {"bytes_per_launch": 800}}
    b.add_traffic(line, {"bytes": 1085, "fetch_kib": 1.0, "fetch_exit_status": -11,
                         "write_exit_status": 0}, None)
    assert line["roofline"]["traffic"] == 1085
    assert line["roofline"]["traffic_ratio"] == pytest.approx(1.085)
    assert line["roofline"]["traffic_ratio_bytes_read"] == pytest.approx(1.3563, abs=1e-4)
    assert line["roofline"]["traffic_counters"]["fetch_exit_status"] == -11
    line = {"roofline": {"bytes_per_launch": 1000, "traffic": None},
            "screened_roofline": {"bytes_per_launch": 800}}
    b.add_traffic(line, None, "FETCH_SIZE pass timed out")
    assert line["roofline"]["traffic"] is None
    assert line["roofline"]["traffic_error"] == "FETCH_SIZE pass timed out"


def test_decode_rooflines_use_the_model_weight_bytes():
    """The line's roofline.frac is the model's weight bytes (fp32 classifier
    as stored) plus K/V over the decode loop's device time; the bytes the
    screened argmax reads are the secondary figure. TinyLlama INT4: 807,518,208
    weight bytes per token."""
    b = bench()
    n, kv = 16, 45056 * sum(5 + i + 1 for i in range(16))
    model_bytes = 807518208 * n + kv
    read_bytes = 615006208 * n + kv
    roof, screened = b.decode_rooflines(model_bytes, read_bytes, 5.495275, "k")
    assert roof["bytes_per_launch"] == 12930023424
    assert roof["frac"] == pytest.approx(12930023424 / 5.495275e-3 / 8e12, abs=1e-4)
    assert roof["frac"] == pytest.approx(0.2941, abs=1e-4)
    assert screened["bytes_per_launch"] == read_bytes
    assert screened["frac"] < roof["frac"]
