"""bench.py's host-side pieces, without a GPU: the refusal of more than one
GPU, and how the roofline picks the dominant kernel's duration out of the
profiler's device records of the decode steps (kernel names as the records
carry them: the mangled names of a rocprofv3 kernel trace of the bench)."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

GEMV = '_ZN2wq12_GLOBAL__N_116gemv_flat_kernelILi{nb}ELi{mm}ELNS0_4WFmtE{f}ELNS0_5XModeE{x}EEEvPKDF16_iiPKvS7_'
RECORDS = {
    GEMV.format(nb=3, mm=1, f=0, x=1): {'us': 6.8, 'per_step': 40.0},    # RMSNorm + QKV
    GEMV.format(nb=3, mm=1, f=0, x=0): {'us': 6.1, 'per_step': 40.0},    # o (+ residual)
    GEMV.format(nb=10, mm=1, f=0, x=1): {'us': 18.1, 'per_step': 40.0},  # RMSNorm + gate_up
    GEMV.format(nb=8, mm=1, f=0, x=2): {'us': 12.5, 'per_step': 40.0},   # SiLU*up + down
    '_ZN2wq12_GLOBAL__N_123decode_attention_kernelILi5ELi2ELi5EEEvPKDF16_': {'us': 7.4, 'per_step': 40.0},
    '_ZN2wq12_GLOBAL__N_129decode_attention_merge_kernelILi32EEEviPKf': {'us': 4.1, 'per_step': 40.0},
    '_ZN2wq12_GLOBAL__N_114lm_head_kernelILi10EEEvPKDF16_S3_iPDF16_': {'us': 231.0, 'per_step': 1.0},
    'lm_head_pick_kernel': {'us': 5.6, 'per_step': 1.0},
}


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / 'bench.py'), '--gpus', '2'], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert 'one GPU' in r.stderr and r.stdout == ''


@pytest.mark.parametrize('name,nb,mm,f,x', [
    ('gemv_flat_kernel<10, 1, W4, RmsNorm>', 10, 1, 0, 1),
    ('gemv_flat_kernel<3, 1, W4>', 3, 1, 0, 0),
    ('gemv_flat_kernel<8, 1, W4, SiluMul>', 8, 1, 0, 2),
    ('gemv_flat_kernel<3, 1, W8, RmsNorm>', 3, 1, 1, 1),
    ('gemv_flat_kernel<10, 4, W4>', 10, 4, 0, 0),
])
def test_report_names_map_to_the_record_names(name, nb, mm, f, x):
    pat = bench.step_record_pattern(name)
    assert pat is not None and pat in GEMV.format(nb=nb, mm=mm, f=f, x=x)
    # no other instantiation carries it (3 is not a prefix of 13, W4 not of W8, ...)
    for other in ((13, mm, f, x), (nb, mm, 1 - f, x), (nb, mm, f, (x + 1) % 3), (nb, mm + 1, f, x)):
        assert pat not in GEMV.format(nb=other[0], mm=other[1], f=other[2], x=other[3])


def test_non_gemv_names_have_no_pattern():
    for name in ('decode_attention_kernel + decode_attention_merge_kernel', 'lm_head_kernel<10> + lm_head_pick_kernel',
                 'gemv_flat_kernel<10, 1, W4, Gelu>', ''):
        assert bench.step_record_pattern(name) is None


def test_in_step_time_of_the_step_kernels():
    gu = bench.step_record_pattern('gemv_flat_kernel<10, 1, W4, RmsNorm>')
    assert bench.in_step_us(RECORDS, (gu,), 40) == pytest.approx(18.1)
    o = bench.step_record_pattern('gemv_flat_kernel<3, 1, W4>')
    assert bench.in_step_us(RECORDS, (o,), 40) == pytest.approx(6.1)   # not the RMSNorm + QKV instantiation
    # attention + merge and the LM head + pick are summed per launch
    assert bench.in_step_us(RECORDS, ('decode_attention_kernel', 'decode_attention_merge_kernel'), 40) == \
        pytest.approx(11.5)
    assert bench.in_step_us(RECORDS, ('lm_head_kernel', 'lm_head_pick_kernel'), 1) == pytest.approx(236.6)


def test_in_step_time_is_none_when_the_records_do_not_fit():
    gu = bench.step_record_pattern('gemv_flat_kernel<10, 1, W4, RmsNorm>')
    assert bench.in_step_us(RECORDS, (gu,), 39) is None        # launch count per step differs
    assert bench.in_step_us({}, (gu,), 40) is None             # no records (an outside profiler held them)
    two = dict(RECORDS)
    two[GEMV.format(nb=10, mm=1, f=0, x=1) + 'clone'] = {'us': 1.0, 'per_step': 40.0}
    assert bench.in_step_us(two, (gu,), 40) is None            # ambiguous: two records match
    assert bench.in_step_us(RECORDS, ('decode_attention_kernel', 'missing_kernel'), 40) is None


def test_in_step_time_is_bounded_by_the_kernels_own_time():
    """Records with the right counts but implausible durations (what the
    profiler returns under rocprofv3: about 1 us per launch) are rejected
    against the kernel's own one-op-graph time; plausible ones pass."""
    gu = bench.step_record_pattern('gemv_flat_kernel<10, 1, W4, RmsNorm>')
    assert bench.in_step_us(RECORDS, (gu,), 40, own_us=19.2) == pytest.approx(18.1)
    assert bench.in_step_us(RECORDS, (gu,), 40, own_us=14.0) == pytest.approx(18.1)   # 1.3x: the step's interleaving
    broken = {k: {'us': 1.3, 'per_step': v['per_step']} for k, v in RECORDS.items()}
    assert bench.in_step_us(broken, (gu,), 40, own_us=21.5) is None
    assert bench.in_step_us(RECORDS, (gu,), 40, own_us=8.0) is None                   # more than 2x
