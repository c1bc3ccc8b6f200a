"""Summaries of rocprofv3 CSV output for the bench workloads.

Two inputs are understood:
  * `<prefix>_kernel_trace.csv` of `rocprofv3 --kernel-trace --output-format csv`
    (one row per dispatch, start/end timestamps in ns);
  * `<prefix>_counter_collection.csv` of `rocprofv3 --pmc <COUNTER> --output-format csv`
    (one row per dispatch and counter).

Library dispatches are mapped to bench.py's launch names by dispatch order:
bench.py first runs every launch once on each of its R rotating buffer sets,
then, launch by launch, `max(5, steps)` repetitions of R back-to-back launches
(the per-launch timing phase), then `warmup` and `steps` steps of all launches.
Only the per-launch phase is summarised, so each figure belongs to one shape.

HBM traffic: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are scaled by what the
same counter reads for a plain copy kernel of known size (bench.py
--calibrate-copy-mib launches torch.neg over that many MiB of float32: the
kernel reads and writes exactly that many bytes), so a factor of 1.0 means the
counter is exact.

Usage:
  python -m deep_gemm.testing.rocprof_summary \
      --bench-json OUT/bench.json --trace OUT/k/x_kernel_trace.csv \
      [--fetch OUT/f/x_counter_collection.csv --write OUT/w/x_counter_collection.csv \
       --copy-mib 1024] [--warmup W --steps S] --md profiles/NAME.md [--json profiles/NAME.json]
"""
import argparse
import csv
import json
import os
import sys

GEMM_KEYS = ('fp8_gemm_1d2d', 'fp8_fp4_gemm', 'fp8_gemm_1d2d_pipe', 'fp8_gemm_masked_stream', 'fp8_gemm_1d1d',
             'fp8_gemm_tinym', 'fp8_gemm_splitk', 'moe_swiglu_cast_kernel')
CAST_KEYS = ('per_token_cast_kernel',)   # the cast workload's kernel (GEMM workloads also cast while setting up)
MOE_DISPATCH_KEYS = ('moe_count_kernel', 'moe_scan_kernel', 'moe_starts_kernel', 'moe_scatter_kernel')
COPY_KEY = 'neg_kernel'
_KEYS = GEMM_KEYS


def _is_gemm(name: str) -> bool:
    return any(k in name for k in _KEYS)


def _short(name: str) -> str:
    """Kernel symbol without the argument list."""
    name = name.replace('(anonymous namespace)::', '').replace('void ', '')
    depth = 0
    for i, ch in enumerate(name):
        if ch == '<':
            depth += 1
        elif ch == '>':
            depth -= 1
        elif ch == '(' and depth == 0:
            return name[:i]
    return name


def phase_slices(num_launches: int, steps: int, rot: int, disp=None):
    """Index ranges, within the library dispatch sequence, of each launch's
    per-launch timing dispatches (repetitions x rotating sets x the launch's
    dispatches per call), and the calls per launch in that phase. `disp[i]` is
    the number of kernels one call of launch i dispatches (2 for a dense column
    split, else 1)."""
    disp = disp or [1] * num_launches
    per = max(5, steps) * rot
    start = rot * sum(disp)
    out = []
    for d in disp:
        out.append(range(start, start + per * d))
        start += per * d
    return out, per


MAX_CLOCK_GHZ = 2.4   # MI355X's highest shader clock


def mfma_utilization(busy_cycles: float, gui_cycles: float, kernel_us: float, simds: int) -> dict:
    """MFMA busy fraction of one call from its counters: busy cycles summed over
    the SIMDs, GRBM_GUI_ACTIVE (GPU-busy clocks, per XCD) of the counter run, and
    the kernel's duration from the trace run. GRBM_GUI_ACTIVE over the traced
    duration is the clock; when that exceeds the chip's 2.4 GHz maximum, the
    counter also counted time outside the kernel (short launches under the
    counter run), so the kernel's clocks are taken as duration x 2.4 GHz instead
    (a lower bound on the busy fraction) and the entry is flagged."""
    clock = gui_cycles / (kernel_us * 1e3)
    over = clock > MAX_CLOCK_GHZ
    cyc = kernel_us * 1e3 * MAX_CLOCK_GHZ if over else gui_cycles
    return {'mfma_busy_frac': busy_cycles / (cyc * simds), 'clock_ghz': min(clock, MAX_CLOCK_GHZ),
            'clock_capped': 1 if over else 0, 'gui_clock_ghz': clock}


def dispatches_per_call(config: str) -> int:
    """Kernels one bench launch dispatches: a dense column split, a contiguous row
    split or the split-K kernel (partials, then the reduction) runs two; a MoE
    dispatch runs its count, scan, (segment starts,) scatter kernels; a launch of
    several library calls (configs joined by ' + ') sums them."""
    if ' + ' in config:
        return sum(dispatches_per_call(c) for c in config.split(' + '))
    if config.startswith('moe_dispatch'):   # count, scan, (starts,) scatter
        return 3 if 'layout=masked' in config else 4
    return 2 if ('split_n=' in config or 'split_m=' in config or ' splits=' in config) else 1


def _workgroups(row) -> int:
    """Workgroups of one dispatch: grid over workgroup size in each dimension the
    trace has (Grid_Size_* counts work-items)."""
    n = 1
    for ax in 'XYZ':
        g, w = row.get(f'Grid_Size_{ax}'), row.get(f'Workgroup_Size_{ax}')
        if g not in (None, '') and w not in (None, ''):
            n *= max(1, int(g) // max(1, int(w)))
    return n


def read_trace(path):
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r['Dispatch_Id']))
    return rows


def read_counters(path, counter):
    """Dispatch_Id -> (kernel name, value) for one counter."""
    out = {}
    for r in csv.DictReader(open(path)):
        if r['Counter_Name'] != counter:
            continue
        did = int(r['Dispatch_Id'])
        name, val = r['Kernel_Name'], float(r['Counter_Value'])
        prev = out.get(did)
        out[did] = (name, val + (prev[1] if prev else 0.0))
    return dict(sorted(out.items()))


def gemm_sequence(items):
    """GEMM entries of (dispatch_id, name, payload) in dispatch order."""
    return [it for it in items if _is_gemm(it[1])]


def summarize(args):
    global _KEYS
    bench = json.loads(open(args.bench_json).read().strip().splitlines()[-1])
    roof = bench['roofline']
    kernels = roof.get('kernel') or []
    if kernels == ['per_token_cast']:
        _KEYS = CAST_KEYS
    elif kernels and all(k.startswith('moe_dispatch') for k in kernels):
        _KEYS = MOE_DISPATCH_KEYS
    else:
        _KEYS = GEMM_KEYS
    names = list(roof['per_launch_us'].keys())
    warmup = args.warmup if args.warmup is not None else bench['warmup']
    steps = args.steps if args.steps is not None else bench['steps']
    rot = bench.get('timing', {}).get('rotating_sets', 1)
    disp = [dispatches_per_call(roof.get('launch_config', {}).get(n, '')) for n in names]
    slices, reps = phase_slices(len(names), steps, rot, disp)

    trace = read_trace(args.trace)
    seq = gemm_sequence([(int(r['Dispatch_Id']), r['Kernel_Name'], r) for r in trace])
    expected = (rot + warmup + steps) * sum(disp) + reps * sum(disp)
    if len(seq) != expected:
        sys.exit(f'expected {expected} library dispatches (warmup {warmup}, steps {steps}, '
                 f'{rot} rotating sets, {len(names)} launches, {sum(disp)} dispatches per step), found {len(seq)}')
    per = []
    for name, sl, d in zip(names, slices, disp):
        rows = [seq[i][2] for i in sl]
        # kernel names in dispatch order (a split call runs two different tiles)
        kern = dict.fromkeys(_short(rows[j]['Kernel_Name']) for j in range(d))
        # one call = d consecutive dispatches: first start to last end
        durs = [(int(rows[c + d - 1]['End_Timestamp']) - int(rows[c]['Start_Timestamp'])) / 1e3
                for c in range(0, len(rows), d)]
        r0 = rows[0]
        grids = [_workgroups(rows[j]) for j in range(d)]
        per.append({'launch': name, 'kernel': ' / '.join(kern), 'calls': len(durs),
                    'avg_us': sum(durs) / len(durs), 'min_us': min(durs), 'max_us': max(durs),
                    'event_us': roof['per_launch_us'][name],
                    'grid': grids[0] if d == 1 else '+'.join(str(g) for g in grids),
                    'vgpr': int(r0['VGPR_Count']), 'agpr': int(r0['Accum_VGPR_Count']),
                    'lds': int(r0['LDS_Block_Size'])})

    traffic = None
    if args.fetch and args.write:
        traffic = {}
        calib = {}
        for counter, path in (('FETCH_SIZE', args.fetch), ('WRITE_SIZE', args.write)):
            vals = read_counters(path, counter)
            copies = [v for _, (n, v) in vals.items() if COPY_KEY in n]
            if not copies:
                sys.exit(f'{path}: no {COPY_KEY} dispatch (run bench.py with --calibrate-copy-mib)')
            known_kib = args.copy_mib * 1024.0
            factor = (sum(copies) / len(copies)) / known_kib
            calib[counter] = {'copy_kib_read': sum(copies) / len(copies), 'copy_kib_known': known_kib,
                              'factor': factor}
            gseq = gemm_sequence([(d, n, v) for d, (n, v) in vals.items()])
            # Under --pmc bench.py runs with the warmup/steps given on the command line.
            psl, preps = phase_slices(len(names), args.pmc_steps, rot, disp)
            exp = (rot + args.pmc_warmup + args.pmc_steps) * sum(disp) + preps * sum(disp)
            if len(gseq) != exp:
                sys.exit(f'{path}: expected {exp} library dispatches, found {len(gseq)}')
            for name, sl, d in zip(names, psl, disp):
                kib = sum(gseq[i][2] for i in sl) / (len(sl) / d)   # per call
                traffic.setdefault(name, {})[counter] = kib * 1024.0 / factor
        traffic = {'per_launch_bytes': {n: {'fetch': round(t['FETCH_SIZE']), 'write': round(t['WRITE_SIZE']),
                                            'total': round(t['FETCH_SIZE'] + t['WRITE_SIZE'])}
                                        for n, t in traffic.items()},
                   'calibration': calib}

    mfma = None
    if args.mfma:
        # MFMA busy cycles summed over every SIMD, and GRBM_GUI_ACTIVE (the
        # kernel's duration in clocks) summed over the XCDs.
        busy = read_counters(args.mfma, 'SQ_VALU_MFMA_BUSY_CYCLES')
        gui = read_counters(args.mfma, 'GRBM_GUI_ACTIVE')
        bseq = gemm_sequence([(d, n, v) for d, (n, v) in busy.items()])
        gseq2 = gemm_sequence([(d, n, v) for d, (n, v) in gui.items()])
        psl, _ = phase_slices(len(names), args.pmc_steps, rot, disp)
        mfma = {}
        for name, sl, p, d in zip(names, psl, per, disp):
            b = sum(bseq[i][2] for i in sl) / (len(sl) / d)   # per call
            cyc = sum(gseq2[i][2] for i in sl) / (len(sl) / d) / args.xcds
            mfma[name] = mfma_utilization(b, cyc, p['avg_us'], args.simds)

    lines = []
    lines.append(f"# {bench['config']['workload']}\n")
    lines.append('Kernel durations from `rocprofv3 --kernel-trace --stats`, per-launch timing phase of '
                 f'bench.py (after a cache flush, {rot} back-to-back launches of one shape on rotating buffer '
                 'sets, repeated), next to the HIP-event average per launch that bench.py measured in the '
                 'same run.\n')
    lines.append('Commands (repository root on the GPU box; `OUT` = an output folder):\n')
    lines.append('```')
    for c in args.command or []:
        lines.append(c)
    lines.append('```\n')
    lines.append('| launch | kernel | grid | VGPR/AGPR | LDS B | calls | rocprof avg us | min | max | '
                 'bench event us |')
    lines.append('|---|---|---|---|---|---|---|---|---|---|')
    for p in per:
        lines.append(f"| {p['launch']} | `{p['kernel']}` | {p['grid']} | {p['vgpr']}/{p['agpr']} | {p['lds']} | "
                     f"{p['calls']} | {p['avg_us']:.1f} | {p['min_us']:.1f} | {p['max_us']:.1f} | "
                     f"{p['event_us']:.1f} |")
    lines.append('')
    tot_r = sum(p['avg_us'] for p in per)
    tot_e = sum(p['event_us'] for p in per)
    lines.append(f'Sum over launches: rocprof {tot_r:.1f} us, bench events {tot_e:.1f} us '
                 f'(ratio {tot_e / tot_r:.3f}).\n')
    lines.append(f"bench.py line: value {bench['value']} {bench['unit']}, roofline achieved "
                 f"{roof['achieved']} {roof['unit']} of {roof['peak']} (frac {roof['frac']}).\n")
    if traffic:
        lines.append('## HBM traffic (FETCH_SIZE / WRITE_SIZE, calibrated)\n')
        for c, v in traffic['calibration'].items():
            lines.append(f"- {c}: copy kernel read {v['copy_kib_read']:.0f} KiB for "
                         f"{v['copy_kib_known']:.0f} KiB moved, factor {v['factor']:.4f}")
        lines.append('')
        lines.append('| launch | fetch MB | write MB | total MB | algorithmic MB | total / algorithmic |')
        lines.append('|---|---|---|---|---|---|')
        algo = roof.get('algorithmic_bytes', {})
        for n, t in traffic['per_launch_bytes'].items():
            a = algo.get(n)
            ratio = f'{t["total"] / a:.2f}' if a else '-'
            lines.append(f"| {n} | {t['fetch'] / 1e6:.1f} | {t['write'] / 1e6:.1f} | {t['total'] / 1e6:.1f} | "
                         f"{(a or 0) / 1e6:.1f} | {ratio} |")
        lines.append('')
    if mfma:
        lines.append('## MFMA utilization (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs))\n')
        lines.append(f'{args.simds} SIMDs, GRBM_GUI_ACTIVE averaged over {args.xcds} XCDs; the clock is '
                     'GRBM_GUI_ACTIVE over the traced kernel time (under the counter run, so approximate). '
                     'Where that exceeds 2.4 GHz (marked *), GRBM_GUI_ACTIVE counted time outside the kernel: '
                     'the clock is taken as 2.4 GHz and MFMA busy is a lower bound.\n')
        lines.append('| launch | MFMA busy | clock GHz | MFMA busy x clock / 2.4 GHz |')
        lines.append('|---|---|---|---|')
        for n, v in mfma.items():
            mark = f" * (GRBM {v['gui_clock_ghz']:.2f})" if v['clock_capped'] else ''
            lines.append(f"| {n} | {100 * v['mfma_busy_frac']:.1f}% | {v['clock_ghz']:.2f}{mark} | "
                         f"{100 * v['mfma_busy_frac'] * v['clock_ghz'] / 2.4:.1f}% |")
        lines.append('')
    os.makedirs(os.path.dirname(os.path.abspath(args.md)), exist_ok=True)
    open(args.md, 'w').write('\n'.join(lines))
    if args.json:
        out = {'workload': bench['config']['workload'],
               'launch_config': roof.get('launch_config', {}),
               'kernel_us': {p['launch']: round(p['avg_us'], 2) for p in per}}
        if traffic:
            out.update(traffic)
        if mfma:
            out['mfma'] = {n: {k: round(x, 4) for k, x in v.items()} for n, v in mfma.items()}
        open(args.json, 'w').write(json.dumps(out, indent=1) + '\n')
    print('\n'.join(lines))


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument('--bench-json', required=True)
    ap.add_argument('--trace', required=True)
    ap.add_argument('--fetch')
    ap.add_argument('--write')
    ap.add_argument('--mfma', help='counter CSV of SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE')
    ap.add_argument('--simds', type=int, default=1024)
    ap.add_argument('--xcds', type=int, default=8)
    ap.add_argument('--copy-mib', type=float, default=1024)
    ap.add_argument('--warmup', type=int)
    ap.add_argument('--steps', type=int)
    ap.add_argument('--pmc-warmup', type=int, default=0)
    ap.add_argument('--pmc-steps', type=int, default=1)
    ap.add_argument('--md', required=True)
    ap.add_argument('--json')
    ap.add_argument('--command', action='append', help='command line to record in the summary')
    summarize(ap.parse_args(argv))


if __name__ == '__main__':
    main()
