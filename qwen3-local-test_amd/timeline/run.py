"""In-kernel timeline of the one-launch decode (k_decode_ld) on the GPU, through the stamped library that
make.py builds: per streaming workgroup the start, the prologue's end, each tile's landing (loader waves) and
take (compute waves), the end of the tile loop, the partial stores and the split record; per combining
workgroup its start, each wave's group staged and summed, and the output. Times are in microseconds from
the first workgroup's start (s_memrealtime, 100 MHz), medians over 10 launches; per XCD the medians of the
loop end and the record.

Usage: python qwen3-local-test_amd/timeline/run.py [pos:n_split:slots ...]   (default 32768:0:16 16384:0:16)
"""
import ctypes
import json
import os
import statistics
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import torch  # noqa: E402

import bench  # noqa: E402

qw = bench.load_package()
qw.LIB_PATH = os.path.join(ROOT, "qwen3-local-test_amd", "_build", "timeline", "libqwattn_timeline.so")
qw.load_library()
plib = ctypes.CDLL(qw.LIB_PATH)
plib.probe_set.argtypes = [ctypes.c_void_p]
TICK = 0.01  # us per s_memrealtime tick (100 MHz)
cases = [tuple(int(x) for x in a.split(":")) for a in (sys.argv[1:] or ["32768:0:16", "16384:0:16"])]
for pos, nsplit, slots in cases:
    wl = bench.Workload(qw, "t", pos, 1, slots, nsplit, "f32", 0.0, seed=1)
    wl.step_events(0, [torch.cuda.Event(enable_timing=True) for _ in range(3)])
    for i in range(8):
        wl.main_only(i % slots)
    torch.cuda.synchronize()
    S, NC = wl.used, bench.NH
    nwg = NC + S * bench.NKV
    buf = torch.zeros(nwg * 4 * 32, dtype=torch.int64, device="cuda")
    plib.probe_set(ctypes.c_void_p(buf.data_ptr()))
    reps = []
    for rep in range(10):
        buf.zero_()
        bench.gpu_sleep(1.0)
        wl.main_only((rep + 5) % slots)
        torch.cuda.synchronize()
        d = buf.cpu().numpy().reshape(nwg, 4, 32)
        st = d[..., :31].astype(np.float64)
        t0 = st[..., 0][st[..., 0] > 0].min()
        reps.append((np.where(st > 0, (st - t0) * TICK, np.nan), (d[NC:, 0, 31] >> 32) & 0xF))
    plib.probe_set(ctypes.c_void_p(0))
    med = lambda x: float(np.nanmedian(x))
    out, per_xcd = [], {}
    for T, xcc in reps:
        C, W = T[:NC], T[NC:]
        land = W[:, 2:, 8:24]
        loop_end = np.nanmax(W[:, :2, 2], axis=1)
        out.append(dict(workgroups_started=med(W[:, 0, 0]), first_tile_landed=med(land[..., 0]),
                        last_tile_landed=med(np.nanmax(land, axis=(1, 2))),
                        last_tile_landed_max=float(np.nanmax(land)), tile_loop_end=med(loop_end),
                        tile_loop_end_max=float(np.nanmax(loop_end)), partials_stored_max=float(np.nanmax(W[:, 0, 3])),
                        record_stored=med(W[:, 0, 4]), record_stored_max=float(np.nanmax(W[:, 0, 4])),
                        combiner_groups_staged=med(np.nanmax(C[:, :, 5], axis=1)),
                        combiner_groups_summed_max=float(np.nanmax(C[:, :, 6])),
                        output_written_max=float(np.nanmax(C[:, 0, 7]))))
        for x in np.unique(xcc):
            sel = xcc == x
            per_xcd.setdefault(int(x), []).append((med(loop_end[sel]), med(W[sel, 0, 4])))
    summ = {k: round(statistics.median([o[k] for o in out]), 2) for k in out[0]}
    xcd = {x: {"tile_loop_end": round(statistics.median([v[0] for v in vs]), 2),
               "record_stored": round(statistics.median([v[1] for v in vs]), 2)} for x, vs in sorted(per_xcd.items())}
    print(json.dumps(dict(pos=pos, splits=S, **summ)), flush=True)
    print(json.dumps({"per_xcd": xcd}), flush=True)
    wl.close()
    del wl
    torch.cuda.empty_cache()
