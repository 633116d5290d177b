"""bench.py's contract on the CPU: one GPU only (a multi-GPU request exits with a message), JSON on stdout."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_multi_gpu_request_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_summarize_trace_and_counters(tmp_path):
    # --summarize reads rocprofv3's CSVs without a GPU: the last N dispatches of the named kernel
    tr = tmp_path / "run_kernel_trace.csv"
    tr.write_text('"Kind","Dispatch_Id","Kernel_Name","Start_Timestamp","End_Timestamp"\n' +
                  "".join(f'"KERNEL_DISPATCH",{i},"{"decode_kernel<128>" if i % 2 else "other"}",{1000 * i},'
                          f'{1000 * i + (2000 if i < 6 else 5000)}\n' for i in range(1, 11)))
    r = subprocess.run([sys.executable, BENCH, "--summarize", str(tr), "--kernel", "decode_kernel", "--last", "2"],
                       capture_output=True, text=True, check=True)
    assert "dispatches summarized: 2 (the last 2 of 5)" in r.stdout
    assert "avg 5.000" in r.stdout  # dispatches 7 and 9: 5 us each
    pc = tmp_path / "run_counter_collection.csv"
    pc.write_text('"Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value"\n'
                  '1,"__amd_rocclr_copyBuffer","FETCH_SIZE",524288\n2,"decode_kernel<128>","FETCH_SIZE",100\n'
                  '3,"decode_kernel<128>","FETCH_SIZE",300\n')
    r = subprocess.run([sys.executable, BENCH, "--summarize", str(pc), "--kernel", "decode_kernel"],
                       capture_output=True, text=True, check=True)
    assert "FETCH_SIZE: avg 200.00" in r.stdout and "copyBuffer (1 GiB copy of the same run) FETCH_SIZE: 524288" in r.stdout
