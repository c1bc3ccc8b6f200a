"""The rocprof summary's mapping of library dispatches to bench.py launches (CPU,
synthetic rocprofv3 CSVs): one dispatch per call, and two for a dense column
split, whose call time runs from the first kernel's start to the second's end."""
import csv
import json

from deep_gemm.testing import rocprof_summary as rs

TRACE_FIELDS = ['Dispatch_Id', 'Kernel_Name', 'Start_Timestamp', 'End_Timestamp', 'Grid_Size_X',
                'Workgroup_Size_X', 'VGPR_Count', 'Accum_VGPR_Count', 'LDS_Block_Size']


def _sequence(rot, warmup, steps, disp):
    """The order bench.py dispatches in: every set of every launch once, then each
    launch's timing phase (max(5, steps) x rot calls), then warmup + steps steps.
    Yields (launch index, dispatch index within the call)."""
    for i, d in enumerate(disp):
        for _ in range(rot):
            yield from ((i, j) for j in range(d))
    for i, d in enumerate(disp):
        for _ in range(max(5, steps) * rot):
            yield from ((i, j) for j in range(d))
    for _ in range(warmup + steps):
        for i, d in enumerate(disp):
            yield from ((i, j) for j in range(d))


def test_split_launch_calls_span_both_dispatches(tmp_path):
    rot, warmup, steps = 2, 1, 1
    names = ['n4096_k7168', 'n7168_k16384']
    configs = {'n4096_k7168': 'fp8_gemm_1d2d v2 kind=normal block_m=256 block_n=256',
               'n7168_k16384': 'fp8_gemm_1d2d v2 kind=normal block_m=256 block_n=256 split_n=4096:256x192'}
    disp = [1, 2]
    # launch 0: one 10 us kernel; launch 1: 7 us, a 1 us gap, then 5 us -> 13 us per call
    kern = {(0, 0): ('fp8_gemm_1d2d_pipe_kernel<256, 256>', 10.0, 256),
            (1, 0): ('fp8_gemm_1d2d_pipe_kernel<256, 256>', 7.0, 256),
            (1, 1): ('fp8_gemm_1d2d_pipe_kernel<256, 192>', 5.0, 256)}
    rows, t, did = [], 0, 0
    fetch_rows, write_rows = [], []
    for i, j in _sequence(rot, warmup, steps, disp):
        name, us, grid = kern[(i, j)]
        rows.append({'Dispatch_Id': did, 'Kernel_Name': name, 'Start_Timestamp': t,
                     'End_Timestamp': t + int(us * 1000), 'Grid_Size_X': grid * 512, 'Workgroup_Size_X': 512,
                     'VGPR_Count': 248, 'Accum_VGPR_Count': 0, 'LDS_Block_Size': 149504})
        t += int(us * 1000) + 1000
        did += 1
    with open(tmp_path / 'trace.csv', 'w', newline='') as f:
        w = csv.DictWriter(f, fieldnames=TRACE_FIELDS)
        w.writeheader()
        w.writerows(rows)
    # counter runs (--steps 1 --warmup 0): 100 KiB per dispatch, plus the copy kernel
    cdid = 0
    for path, counter in ((tmp_path / 'fetch.csv', 'FETCH_SIZE'), (tmp_path / 'write.csv', 'WRITE_SIZE')):
        with open(path, 'w', newline='') as f:
            w = csv.DictWriter(f, fieldnames=['Dispatch_Id', 'Kernel_Name', 'Counter_Name', 'Counter_Value'])
            w.writeheader()
            w.writerow({'Dispatch_Id': cdid, 'Kernel_Name': 'neg_kernel', 'Counter_Name': counter,
                        'Counter_Value': 1024.0 * 1024})
            for k, (i, j) in enumerate(_sequence(rot, 0, 1, disp)):
                w.writerow({'Dispatch_Id': cdid + 1 + k, 'Kernel_Name': kern[(i, j)][0], 'Counter_Name': counter,
                            'Counter_Value': 100.0})
    bench = {'value': 1.0, 'unit': 'TFLOPS', 'warmup': warmup, 'steps': steps, 'config': {'workload': 'synthetic'},
             'timing': {'rotating_sets': rot},
             'roofline': {'per_launch_us': {'n4096_k7168': 10.5, 'n7168_k16384': 13.5}, 'launch_config': configs,
                          'achieved': 1.0, 'unit': 'TFLOP/s', 'peak': 5000.0, 'frac': 0.0002,
                          'algorithmic_bytes': {'n4096_k7168': 102400, 'n7168_k16384': 204800}}}
    (tmp_path / 'bench.json').write_text(json.dumps(bench) + '\n')
    rs.main(['--bench-json', str(tmp_path / 'bench.json'), '--trace', str(tmp_path / 'trace.csv'),
             '--fetch', str(tmp_path / 'fetch.csv'), '--write', str(tmp_path / 'write.csv'),
             '--copy-mib', '1024', '--md', str(tmp_path / 'out.md'), '--json', str(tmp_path / 'out.json')])
    out = json.loads((tmp_path / 'out.json').read_text())
    assert out['kernel_us'] == {'n4096_k7168': 10.0, 'n7168_k16384': 13.0}
    # per call: one dispatch of 100 KiB, or two
    assert out['per_launch_bytes']['n4096_k7168']['fetch'] == 100 * 1024
    assert out['per_launch_bytes']['n7168_k16384']['write'] == 200 * 1024
    md = (tmp_path / 'out.md').read_text()
    assert '| 256+256 |' in md and '| 10 |' in md   # grids of both dispatches; 10 calls in the phase


def test_dispatches_per_call():
    assert rs.dispatches_per_call('fp8_gemm_1d2d v2 kind=normal block_m=256 block_n=256') == 1
    assert rs.dispatches_per_call('fp8_gemm_1d2d v2 kind=normal block_m=256 block_n=256 split_n=4096:256x192') == 2
    assert rs.dispatches_per_call('fp8_gemm_1d2d v2 kind=m_grouped_contiguous block_m=256 block_n=256 '
                                  'split_m=32768:128x128') == 2


def test_dispatches_per_call_split_k_and_joined_calls():
    assert rs.dispatches_per_call('fp8_gemm_1d2d v10 kind=normal block_m=64 block_n=64 m=64 n=2112 k=7168 '
                                  'groups=1 splits=7x8') == 2
    assert rs.dispatches_per_call('fp8_gemm_1d2d v2 kind=m_grouped_contiguous block_m=256 block_n=256 + '
                                  'moe_swiglu_cast gran_k=128 m=33408 n=2048') == 2


def test_dispatches_per_call_moe_dispatch():
    """count, scan, segment starts and scatter; the masked layout has no starts."""
    assert rs.dispatches_per_call('moe_dispatch layout=contiguous experts=256 t=4096 k=8 kdim=7168') == 4
    assert rs.dispatches_per_call('moe_dispatch layout=psum experts=256 t=4096 k=8 kdim=7168') == 4
    assert rs.dispatches_per_call('moe_dispatch layout=masked experts=16 t=512 k=8 kdim=7168') == 3


def test_mfma_clock_capped_at_chip_maximum():
    """GRBM_GUI_ACTIVE over the traced duration gives the clock; above 2.4 GHz the
    counter included time outside the kernel, so the busy fraction is taken over
    duration x 2.4 GHz (a lower bound) and flagged; below it is used as is."""
    simds = 1024
    # 10 us kernel, 2.0 GHz: 20000 cycles; half of them MFMA-busy on every SIMD
    v = rs.mfma_utilization(0.5 * 20000 * simds, 20000, 10.0, simds)
    assert abs(v['mfma_busy_frac'] - 0.5) < 1e-12 and abs(v['clock_ghz'] - 2.0) < 1e-12 and not v['clock_capped']
    # 10 us kernel whose GRBM count implies 3.28 GHz: capped at 2.4 GHz
    v = rs.mfma_utilization(0.5 * 24000 * simds, 32800, 10.0, simds)
    assert v['clock_capped'] and abs(v['clock_ghz'] - 2.4) < 1e-12 and abs(v['gui_clock_ghz'] - 3.28) < 1e-12
    assert abs(v['mfma_busy_frac'] - 0.5) < 1e-12
