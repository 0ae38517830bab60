"""Host-side arithmetic of bench.py (no GPU): the algorithmic byte counts the
roofline is priced on, their split over the kernels, and the folding of
rocprofv3 counter passes into per-launch HBM traffic."""
from __future__ import annotations

import csv
import json

import pytest

import bench

# det: N_all = 6 x 118 x 32 x 88, 360 x 360 x 1 cells, C = 80 fp32; N_kept and
# the occupied cells of the synthetic rig
DET = dict(n_all=1_993_728, n_kept=1_774_050, n_occ=45_826, cells=129_600, C=80)
SEG = dict(n_all=1_993_728, n_kept=1_716_944, n_occ=39_207, cells=65_536, C=80)


def test_alg_bytes_det_closed_form():
    fwd, bwd = bench.alg_bytes(**DET)
    # geometry read (3 fp32) + kept rows read + dense BEV written
    assert fwd == 12 * 1_993_728 + 320 * 1_774_050 + 320 * 129_600 == 633_092_736
    # occupied gradient rows read + full feature gradient written
    assert bwd == 320 * 45_826 + 320 * 1_993_728 == 652_657_280
    # the 60% target of the det row: 1,285.8 MB at 4.8 TB/s
    assert round((fwd + bwd) / 1e6, 1) == 1285.8
    assert round((fwd + bwd) / (0.6 * bench.HBM_PEAK_GBS * 1e3), 1) == 267.9


def test_alg_bytes_seg_and_bf16_element_size():
    fwd, bwd = bench.alg_bytes(**SEG)
    assert round((fwd + bwd) / 1e6, 1) == 1244.9
    f2, b2 = bench.alg_bytes(**DET, s=2)
    assert f2 == 12 * DET['n_all'] + 160 * DET['n_kept'] + 160 * DET['cells']
    assert b2 == 160 * DET['n_occ'] + 160 * DET['n_all']


@pytest.mark.parametrize('case', [DET, SEG])
def test_kernel_bytes_partition_the_path(case):
    """Every algorithmic term is charged to exactly one kernel: the five
    kernels' shares add up to the path's bytes, and the dominant kernel's
    share is the kept rows alone (keys and cell rows are auxiliary)."""
    fwd, bwd = bench.alg_bytes(**case)
    names = ('quantize_geom', 'accum_rows', 'rows_to_bev', 'bev_to_rows', 'gather_rows')
    assert sum(bench.kernel_alg_bytes(n, **case) for n in names) == fwd + bwd
    assert bench.kernel_alg_bytes('accum_rows', **case) == 4 * case['C'] * case['n_kept']
    assert bench.kernel_aux_bytes('accum_rows', **case) == (8 * case['n_kept']
                                                            + 4 * case['C'] * case['n_occ'])
    for n in ('radix_scan', 'radix_scatter', 'bucket_sort'):
        assert bench.kernel_alg_bytes(n, **case) is None  # pure overhead


def _write_pmc(path, counter, rows):
    fields = ['Dispatch_Id', 'Kernel_Name', 'Counter_Name', 'Counter_Value']
    with open(path, 'w', newline='') as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for i, (name, v) in enumerate(rows):
            w.writerow({'Dispatch_Id': i + 1, 'Kernel_Name': name, 'Counter_Name': counter,
                        'Counter_Value': v})


def test_fold_pmc_scales_by_the_calibrators(tmp_path, monkeypatch):
    """FETCH_SIZE is scaled so the read-only sum reads 512 MiB and WRITE_SIZE
    so the copy writes 512 MiB; a kernel's traffic is the sum of its scaled
    per-dispatch means; other kernels (torch's) are ignored."""
    monkeypatch.setattr(bench, 'ROOT', tmp_path)
    (tmp_path / 'profiles').mkdir()
    kib = bench.CALIBRATOR_BYTES / 1024
    accum = 'void (anonymous namespace)::accum_pipe_kernel<F32, 5, 2, 2>(...)'
    gather = 'void (anonymous namespace)::gather_rows_kernel<u32x4, true>(...)'
    fetch = [(accum, 1000.0), (accum, 1200.0), (gather, 50.0), ('void at::fill_kernel', 9e9),
             ('copyBuffer', kib / 2), ('reduce_kernel<sum>', kib / 2)]  # reads half: factor 2
    write = [(accum, 10.0), (accum, 10.0), (gather, 4000.0), ('copyBuffer', kib)]  # factor 1
    _write_pmc(tmp_path / 'f.csv', 'FETCH_SIZE', fetch)
    _write_pmc(tmp_path / 'w.csv', 'WRITE_SIZE', write)
    bench.fold_pmc(tmp_path / 'f.csv', tmp_path / 'w.csv', 'unit')
    out = json.loads((tmp_path / 'profiles' / 'traffic_unit.json').read_text())
    cal = out['calibration']
    assert cal['fetch_factor_read_only'] == 2.0 and cal['write_factor'] == 1.0
    k = out['kernels']
    assert set(k) == {'accum_rows', 'gather_rows'}
    assert k['accum_rows']['fetch_kib'] == 1100.0
    assert k['accum_rows']['traffic_bytes'] == int((1100.0 * 2 + 10.0) * 1024)
    assert k['gather_rows']['traffic_bytes'] == int((50.0 * 2 + 4000.0) * 1024)


def test_fold_pmc_needs_the_calibrators(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, 'ROOT', tmp_path)
    (tmp_path / 'profiles').mkdir()
    _write_pmc(tmp_path / 'f.csv', 'FETCH_SIZE', [('accum_pipe_kernel', 1.0)])
    _write_pmc(tmp_path / 'w.csv', 'WRITE_SIZE', [('accum_pipe_kernel', 1.0)])
    with pytest.raises(SystemExit, match='calibrator'):
        bench.fold_pmc(tmp_path / 'f.csv', tmp_path / 'w.csv', 'unit')


def test_cpu_threads_follow_the_environment(monkeypatch):
    monkeypatch.setenv('OMP_NUM_THREADS', '1')
    n, aff, src = bench.cpu_threads()
    assert (n, src) == (1, 'OMP_NUM_THREADS') and aff >= 1
    monkeypatch.delenv('OMP_NUM_THREADS')
    n, aff, src = bench.cpu_threads()
    assert src == 'affinity' and n == aff


@pytest.mark.parametrize('mode', ['bench', 'ceiling'])
def test_op_level_config_only_in_kernels_mode(monkeypatch, capsys, mode):
    """The op-level bf16 configuration runs under --mode kernels (counter
    passes) and --mode configs only; the headline modes refuse it before the
    package or the GPU is touched."""
    monkeypatch.setattr('sys.argv', ['bench.py', '--mode', mode, '--config', 'bf16'])
    monkeypatch.setattr(bench.__graft_entry__, 'load_package',
                        lambda: pytest.fail('the package was loaded'))
    with pytest.raises(SystemExit) as e:
        bench.main()
    assert e.value.code == 2
    assert 'op-level configuration' in capsys.readouterr().err
