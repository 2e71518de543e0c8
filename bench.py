"""Benchmark of the semi-naive relational core on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload c4|c1|c1j|c1h|c2|c2u|c3|c4j|c4h|c5|c5j|tcs|tcs_crit|tcs_j|copy|c5full]
                    [--no-extra] [--no-cpu-baseline]

Default workload is BASELINE.json configs[3] (C4), the metric's lead quantity:
the semi-naive transitive closure of a seeded G(32768, 98304) digraph, run to
fixpoint on inputs already resident in HBM.  One step is one whole fixpoint,
the emit of the ~9.5 x 10^8 sorted closure tuples included; `ms_per_step` is
the fixpoint wall time and `value` is closure tuples per second of it.

With the default workload the same line carries the other configs under
`configs` (c1: TC on G(1000, 5000); c2: R(a,b) join S(b,c), project, sort +
dedup at 2^24 rows a side; c3: sort + dedup of 2^28 packed tuples; c5: Andersen
points-to at 10,000 variables), each with its own timing, roofline and CPU
baseline.  c5_stated is C5 at its stated 500,000 variables, run once for its outcome
(the reference's u32 join-row limit trips in the first recursive iteration).
c1j / c4j / c5j force the join route and c1h / c4h the hash-set route;
tcs / tcs_crit are closures over 2^20 vertices whose ids are spread over u32
(the hash-set route, AUTO's choice there) and tcs_j is tcs on the join route;
c2u is the unfused join -> sort -> dedup sequence; copy is the counter
calibration kernel; c5full runs C5 at its stated 500,000 variables once and
reports its outcome (the library fails closed at the reference's 2^32-1 join
row limit).

Every `roofline` object describes the kernel kind with the largest share of
device time in the timed steps, timed live with HIP events on the library's
stream (algorithmic bytes / average launch time).  `cpu_baseline` is the CPU
oracle (oracle/oracle.c) with every host thread and single-threaded.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

METRIC = "semi-naive fixpoint wall time + join/sort tuples/s; % of HBM peak, 1 MI355X"
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_workload(name: str, p):
    """Returns (step_fn, units_per_step, unit_desc, config, checker_inputs)."""
    from xlog_amd import datagen, tc_plan, andersen_plan, pack

    if name in ("c2", "c2u"):
        cfg = datagen.C2
        t = time.perf_counter()
        r_a, r_b, s_b, s_c = datagen.zipf_join(cfg["n_r"], cfg["n_s"], cfg["n_keys"], cfg["zipf_s"], datagen.seed_for(2))
        log(f"c2 inputs generated in {time.perf_counter() - t:.1f}s")
        R = p.create_buffer_from_u32_columns([r_a, r_b])
        S = p.create_buffer_from_u32_columns([s_b, s_c])
        state = {}

        if name == "c2":
            # fused operator: the join is emitted in (a, c) order, no sort of the 2^28-row output
            def step():
                d = p.join_project_dedup(R, S, 1, 0, [0, 3])
                state["out_rows"] = d.num_rows()
        else:
            # unfused: join + project (bag of ~2^28 rows), then radix sort + unique
            def step():
                j = p.join_project(R, S, 1, 0, [0, 3])
                d = p.dedup_full_row(j)
                state["join_rows"] = j.num_rows()
                state["out_rows"] = d.num_rows()

        units = cfg["n_r"] + cfg["n_s"]
        how = ("fused order-preserving join+project+dedup" if name == "c2"
               else "join+project, then radix sort + unique of the join output")
        config = {"workload": f"c2: R(a,b) join S(b,c) on b, project (a,c), sort + dedup ({how})",
                  "rows_r": cfg["n_r"], "rows_s": cfg["n_s"], "keys": cfg["n_keys"], "zipf_s_probe_side": cfg["zipf_s"],
                  "build_side_keys": "uniform", "seed": datagen.seed_for(2)}
        return step, units, "input tuples (|R|+|S|)", config, (r_a, r_b, s_b, s_c), state
    if name == "c3":
        n = datagen.C3["n"]
        t = time.perf_counter()
        keys = datagen.dup_tuples(n, datagen.seed_for(3))
        log(f"c3 inputs generated in {time.perf_counter() - t:.1f}s")
        K = p.create_buffer_from_packed(keys)
        state = {}

        def step():
            d = p.dedup_full_row(K)
            state["out_rows"] = d.num_rows()

        config = {"workload": "c3: radix sort + dedup of 2^28 packed u64 tuples, 30% exact duplicates",
                  "tuples": n, "seed": datagen.seed_for(3)}
        return step, n, "input tuples", config, (keys,), state
    if name in ("c1", "c4", "c1j", "c4j", "c1h", "c4h", "tcs", "tcs_crit", "tcs_j"):
        # c1j / c4j: the same closure forced onto the join route (per iteration: delta join edge, radix
        # sort, unique and not-in-R selection, merge into R); c1h / c4h onto the hash-set route (one fused
        # expand + insert pass per iteration) instead of the bitmap route AUTO picks.  tcs / tcs_crit: G(2^20, m)
        # digraphs with ids spread over the u32 range (beyond the bit-matrix domain: AUTO takes the hash
        # route; tcs_j forces the join route)
        from xlog_amd import ROUTE_AUTO, ROUTE_HASH, ROUTE_JOIN
        route = {"j": ROUTE_JOIN, "h": ROUTE_HASH}.get(name[-1], ROUTE_AUTO)
        if name.startswith("tcs"):
            cfg = datagen.TCS_CRIT if name == "tcs_crit" else datagen.TCS
            cid = 6
        else:
            cfg = datagen.C1 if name.startswith("c1") else datagen.C4
            cid = 1 if name.startswith("c1") else 4
        src, dst = datagen.random_digraph(cfg["n_vertices"], cfg["n_edges"], datagen.seed_for(cid))
        graph = (src, dst)  # the CPU baseline's BFS takes the dense ids (same closure up to relabelling)
        if name.startswith("tcs"):
            src, dst = datagen.sparse_ids(src), datagen.sparse_ids(dst)
        E = p.create_buffer_from_u32_columns([src, dst])
        state = {}

        def step():
            outs, st = p.fixpoint(tc_plan(), [E, None], route=route)
            state["out_rows"] = outs[1].num_rows()
            state["iterations"] = st["iterations"]
            state["delta_sizes"] = st["delta_sizes"]
            state["route"] = st["route"]
            state["host_waits"] = st["host_waits"]

        config = {"workload": f"{name}: semi-naive transitive closure, G(n,m) digraph"
                              + (" with ids spread over u32" if name.startswith("tcs") else "")
                              + {ROUTE_JOIN: " (join route)", ROUTE_HASH: " (hash-set route)"}.get(route, ""),
                  "vertices": cfg["n_vertices"], "edges": cfg["n_edges"], "seed": datagen.seed_for(cid)}
        return step, None, "closure tuples", config, (graph, cfg["n_vertices"]), state
    if name == "copy":
        # calibration: k_project over 2^28 packed rows reads 8 B and writes 8 B per row
        n = 1 << 28
        K = p.create_buffer_from_packed(np.arange(n, dtype=np.uint64))
        state = {}

        def step():
            o = p.project(K, [1, 0])
            state["out_rows"] = o.num_rows()

        config = {"workload": "copy: column swap of 2^28 packed rows (16 B/row), counter calibration", "rows": n}
        return step, n, "rows", config, None, state
    if name in ("c5", "c5j"):
        # BASELINE's literal C5 (500,000 variables) grows |pointsTo| like V^2 (~10^10 tuples, past the
        # reference's u32 row cap): the bench runs the same generator at 10,000 variables / 40,000 facts
        cfg = dict(datagen.C5, n_vars=10_000, n_facts=40_000)
        f = datagen.andersen(cfg["n_vars"], cfg["n_facts"], cfg["alpha"], datagen.seed_for(5))
        rels = [p.create_buffer_from_u32_columns(list(f[k])) for k in ("assign", "addressOf", "load", "store")]
        state = {}
        from xlog_amd import ROUTE_AUTO, ROUTE_JOIN
        route = ROUTE_JOIN if name == "c5j" else ROUTE_AUTO

        def step():
            outs, st = p.fixpoint(andersen_plan(), rels + [None], route=route)
            state["out_rows"] = outs[4].num_rows()
            state["iterations"] = st["iterations"]
            state["delta_sizes"] = st["delta_sizes"]
            state["route"] = st["route"]
            state["host_waits"] = st["host_waits"]

        def same_sample():
            # the GPU on the instance the CPU baseline runs (5,000 variables), for a like-for-like comparison
            g = datagen.andersen(5000, 20000, cfg["alpha"], datagen.seed_for(5))
            r5 = [p.create_buffer_from_u32_columns(list(g[k])) for k in ("assign", "addressOf", "load", "store")]
            p.fixpoint(andersen_plan(), r5 + [None])
            p.synchronize()
            t = time.perf_counter()
            for _ in range(5):
                outs, _ = p.fixpoint(andersen_plan(), r5 + [None])
            p.synchronize()
            return {"gpu_5000_vars_ms": (time.perf_counter() - t) * 1000.0 / 5, "gpu_5000_vars_tuples": outs[4].num_rows()}

        if name == "c5":
            state["_extra"] = same_sample
        config = {"workload": "c5 scaled: Andersen points-to, 4 rules"
                              " (the stated 500,000 variables fail closed: c5_stated)"
                              + (" (join route)" if name == "c5j" else ""), **cfg,
                  "seed": datagen.seed_for(5)}
        return step, None, "pointsTo tuples", config, f, state
    raise SystemExit(f"unknown workload {name}")


def cpu_baseline(name: str, inputs, budget_s: float = 30.0):
    """CPU oracle (C, oracle/oracle.c) on this host: `value` with every OpenMP thread
    (OMP_NUM_THREADS, or the host's cores) on the workload or a bounded sample of it, and
    `single_thread` on a smaller sample, both stated."""
    import oracle
    from xlog_amd import pack, tc_plan

    threads = oracle.max_threads()

    def timed(fn, t, warmup=False):
        # warmup: one untimed call first, so multi-GB first-touch page faults are not timed
        # (the GPU side is timed after warm-up steps as well)
        oracle.set_threads(t)
        try:
            if warmup:
                fn()
            t0 = time.perf_counter()
            res = fn()
            return res, time.perf_counter() - t0
        finally:
            oracle.set_threads(1)

    def entry(value, unit, cores, sample):
        return {"value": value, "unit": unit, "cores": cores, "kind": "port", "sample": sample}

    if name in ("c2", "c2u"):
        r_a, r_b, s_b, s_c = inputs
        r = pack(s_b, s_c)
        l_all = pack(r_a, r_b)
        n_r = 1 << 22

        def run(l):
            return oracle.sort_dedup(oracle.join_project(l, r, 1, 0, 0, 3))
        out, dt = timed(lambda: run(l_all), threads, warmup=True)
        out1, dt1 = timed(lambda: run(l_all[:n_r]), 1, warmup=True)
        res = entry((len(l_all) + len(r)) / dt, "tuples/s", threads,
                    f"full config: R join S, project + sort + dedup -> {len(out)} tuples in {dt:.2f}s "
                    f"(after one untimed run)")
        res["single_thread"] = entry((n_r + len(r)) / dt1, "tuples/s", 1,
                                     f"first {n_r} rows of R with all of S -> {len(out1)} tuples in {dt1:.2f}s")
        return res
    if name == "c3":
        (keys,) = inputs
        n1 = 1 << 25
        u, dt = timed(lambda: oracle.sort_dedup(keys), threads, warmup=True)
        u1, dt1 = timed(lambda: oracle.sort_dedup(keys[:n1]), 1, warmup=True)
        res = entry(len(keys) / dt, "tuples/s", threads, f"full config: sort + dedup of {len(keys)} -> {len(u)} in {dt:.2f}s")
        res["single_thread"] = entry(n1 / dt1, "tuples/s", 1, f"first {n1} tuples -> {len(u1)} in {dt1:.2f}s")
        return res
    if name == "c5":
        # the semi-naive oracle on the 5,000-variable instance of the same generator
        from xlog_amd import andersen_plan, datagen
        f = datagen.andersen(5000, 20000, 1.5, datagen.seed_for(5))
        rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")] + [None]
        (outs, it, _), dt = timed(lambda: oracle.seminaive(andersen_plan(), rels), threads)
        (outs1, _, _), dt1 = timed(lambda: oracle.seminaive(andersen_plan(), rels), 1)
        smp = f"5,000 variables / 20,000 facts (the bench runs 10,000 / 40,000): {len(outs[4])} tuples, {it} iterations"
        res = entry(len(outs[4]) / dt, "pointsTo tuples/s", threads, f"{smp} in {dt:.2f}s")
        res["single_thread"] = entry(len(outs1[4]) / dt1, "pointsTo tuples/s", 1, f"same instance in {dt1:.2f}s")
        return res
    if name in ("c1", "c1j", "c1h"):
        (src, dst), _ = inputs
        (outs, it, _), dt = timed(lambda: oracle.seminaive(tc_plan(), [pack(src, dst), None]), threads)
        (outs1, _, _), dt1 = timed(lambda: oracle.seminaive(tc_plan(), [pack(src, dst), None]), 1)
        res = entry(len(outs[1]) / dt, "tuples/s", threads,
                    f"full config, semi-naive oracle: {len(outs[1])} tuples, {it} iterations in {dt:.2f}s")
        res["single_thread"] = entry(len(outs1[1]) / dt1, "tuples/s", 1, f"same in {dt1:.2f}s")
        return res
    if name in ("c4", "c4j", "c4h") or name.startswith("tcs"):
        (src, dst), nv = inputs
        # the semi-naive oracle over ~10^9 tuples takes far longer than the budget:
        # time the BFS closed form (closure size from every source) instead
        res_mt, dt = timed(lambda: oracle.bfs_tc(nv, src, dst, want_relation=False, digest=False), threads)
        if name.startswith("tcs"):  # a 1-thread run of the whole closure would take minutes: report the threaded one
            return entry(res_mt["total"] / dt, "tuples/s", threads,
                         f"BFS-layer closure from all sources (closed form, not the semi-naive loop): "
                         f"{res_mt['total']} tuples in {dt:.2f}s")
        res_1, dt1 = timed(lambda: oracle.bfs_tc(nv, src, dst, want_relation=False, digest=False), 1)
        res = entry(res_mt["total"] / dt, "tuples/s", threads,
                    f"BFS-layer closure from all sources (closed form, not the semi-naive loop): "
                    f"{res_mt['total']} tuples in {dt:.2f}s")
        res["single_thread"] = entry(res_1["total"] / dt1, "tuples/s", 1, f"same in {dt1:.2f}s")
        return res
    return None


def measure(name: str, p, steps: int, warmup: int, with_cpu: bool) -> dict:
    """Warm-up, then `steps` timed steps of one workload with live kernel timing;
    returns the per-config record (timing, roofline, kernels, result, CPU baseline)."""
    step, units, unit_desc, config, inputs, state = make_workload(name, p)
    log(f"workload {name}: warmup {warmup}")
    for _ in range(warmup):
        step()
    p.synchronize()
    # The wall clock runs without kernel instrumentation: the HIP events that
    # bracket each profiled launch add about 10 us of launch gap apiece (seen in
    # kernel traces), which is measurement overhead, not work.  The same
    # `steps` steps then run again with the events on, for the live per-kernel
    # durations that the roofline and the kernel table use.
    log(f"workload {name}: timing {steps} steps")
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    p.synchronize()
    t1 = time.perf_counter()
    log(f"workload {name}: {steps} more steps with per-kernel HIP events")
    p.profile_reset()
    p.profile_enable(True)
    tp0 = time.perf_counter()
    for _ in range(steps):
        step()
    p.synchronize()
    tp1 = time.perf_counter()
    p.profile_enable(False)
    prof = p.profile_read()
    # the same-sample GPU figure accompanies the CPU baseline (and stays out of profiler runs without it)
    same_sample = state.pop("_extra", None)
    extra = same_sample() if (same_sample and with_cpu) else {}
    ms = (t1 - t0) * 1000.0 / max(1, steps)
    if units is None:
        units = state.get("out_rows", 0)
    value = units / (ms / 1000.0) if ms > 0 else 0.0

    # dominant kernel: the kind with the largest share of device time in the timed steps
    dname, d = max(prof.items(), key=lambda kv: kv[1]["total_ms"])
    avg_ms = d["total_ms"] / max(1, d["launches"])
    bytes_per_launch = d["algo_bytes"] / max(1, d["launches"])
    achieved = (bytes_per_launch / (avg_ms / 1000.0)) / 1e9 if avg_ms > 0 else 0.0
    # HBM traffic comes from rocprofv3 FETCH_SIZE / WRITE_SIZE runs kept under profiles/, not from this run
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": dname,
                "launches_per_step": d["launches"] / max(1, steps), "avg_launch_ms": round(avg_ms, 4),
                "algo_bytes_per_launch": bytes_per_launch}
    # the whole step against the same peak: every instrumented kernel's algorithmic bytes per step over the
    # uninstrumented wall time of a step (kernels outside the instrumented kinds add bytes not counted here)
    step_bytes = sum(v["algo_bytes"] for v in prof.values()) / max(1, steps)
    step_gbs = step_bytes / (ms / 1000.0) / 1e9 if ms > 0 else 0.0
    step_roofline = {"algo_bytes_per_step": step_bytes, "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4)}
    kernels = {k: {"launches": v["launches"], "total_ms": round(v["total_ms"], 3),
                   "algo_GBps": round(v["algo_bytes"] / (v["total_ms"] / 1000.0) / 1e9, 1) if v["total_ms"] else None}
               for k, v in prof.items() if v["launches"]}
    cpu = None
    if with_cpu:
        log(f"workload {name}: cpu baseline (oracle, bounded sample)")
        cpu = cpu_baseline(name, inputs)
    result = {k: v for k, v in state.items() if k != "delta_sizes"}
    if "delta_sizes" in state:
        result["delta_sizes"] = state["delta_sizes"]
    result.update(extra)
    return {"workload": name, "value": value, "unit": "tuples/s", "value_counts": unit_desc, "ms_per_step": ms,
            "ms_per_step_with_kernel_events": (tp1 - tp0) * 1000.0 / max(1, steps), "steps": steps, "warmup": warmup,
            "config": config, "roofline": roofline, "step_roofline": step_roofline, "cpu_baseline": cpu,
            "kernels": kernels, "result": result}


def run_c5full(p, max_join_rows: int = (1 << 32) - 1) -> dict:
    """BASELINE's literal C5 (500,000 variables / 2,000,000 facts) on the join route with the reference's
    u32 join-row limit (relational.rs:4550-4555): the outcome (converged, or the failure with the iteration
    and the bag size that tripped it), plus the size of rule 2's first-iteration output, a lower bound of
    |pointsTo| computed by the fused join+project+dedup."""
    from xlog_amd import XlogError, andersen_plan, datagen

    cfg = datagen.C5
    t = time.perf_counter()
    f = datagen.andersen(cfg["n_vars"], cfg["n_facts"], cfg["alpha"], datagen.seed_for(5))
    log(f"c5full inputs generated in {time.perf_counter() - t:.1f}s")
    rels = [p.create_buffer_from_u32_columns(list(f[k])) for k in ("assign", "addressOf", "load", "store")]
    out = {"workload": "c5full: Andersen points-to at 500,000 variables / 2,000,000 facts (BASELINE configs[4])",
           **cfg, "seed": datagen.seed_for(5), "max_join_rows": max_join_rows}
    p.synchronize()
    t0 = time.perf_counter()
    try:
        outs, st = p.fixpoint(andersen_plan(), rels + [None], max_join_rows=max_join_rows)
        out.update(outcome="converged", tuples=outs[4].num_rows(), iterations=st["iterations"],
                   delta_sizes=st["delta_sizes"], route=st["route"])
    except XlogError as e:
        st = getattr(e, "stats", {})
        out.update(outcome=f"failed closed: status {e.status}", message=str(e),
                   iterations_reached=st.get("iterations"), delta_sizes=st.get("delta_sizes"), route=st.get("route"))
    p.synchronize()
    out["seconds"] = time.perf_counter() - t0
    if not max_join_rows:
        return out
    # rule 2 of the first iteration alone: {(v, o) : assign(v, w), addressOf(w, o)} (the seed delta is addressOf)
    t0 = time.perf_counter()
    r2 = p.join_project_dedup(rels[0], rels[1], 1, 0, [0, 3])
    p.synchronize()
    out["rule2_first_iteration_tuples"] = r2.num_rows()
    out["rule2_seconds"] = time.perf_counter() - t0
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline workload only (no per-config entries)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus above 1 is not supported",
                          "n_gpus": args.gpus}))
        return 2

    from xlog_amd import HipKernelProvider

    p = HipKernelProvider(0)
    if args.workload in ("c5full", "c5full_nolimit"):
        # c5full_nolimit: the same without the join-row limit (chunked join steps), for its measured outcome
        r = run_c5full(p, 0 if args.workload == "c5full_nolimit" else (1 << 32) - 1)
        print(json.dumps({"metric": METRIC, "value": None, "n_gpus": 1, "result": r}))
        p.close()
        return 0
    head = measure(args.workload, p, args.steps, args.warmup, not args.no_cpu_baseline)
    p.trim()
    extras = {}
    if args.workload == "c4" and not args.no_extra:
        # the other configs of BASELINE.json, each with its own timing and roofline (a few steps each)
        for name, k, w in (("c1", 20, 3), ("c2", 10, 3), ("c3", 3, 1), ("c5", 5, 2)):
            extras[name] = measure(name, p, k, w, not args.no_cpu_baseline)
            p.trim()
        # C5 at its stated size: its outcome (the fail-closed join-row limit, as the reference), once
        extras["c5_stated"] = run_c5full(p)
        p.trim()

    out = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "tuples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "ms_per_step_with_kernel_events": head["ms_per_step_with_kernel_events"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic (seeded generators, xlog_amd/csrc/datagen.c)",
        "config": {**head["config"], "value_counts": head["value_counts"], "parallelism": "single GPU"},
        "roofline": head["roofline"],
        "step_roofline": head["step_roofline"],
        "cpu_baseline": head["cpu_baseline"],
        "kernels": head["kernels"],
        "result": head["result"],
    }
    if extras:
        out["configs"] = {k: {kk: vv for kk, vv in v.items() if kk != "workload"} for k, v in extras.items()}
    print(json.dumps(out))
    p.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
