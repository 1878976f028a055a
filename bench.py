"""Benchmark: INT8 MoE decode at batch 1 on one MI355X.

Workload: 11 stacked DeepSeek3B-MoE layers (hidden 1280, 64 routed experts of gate_up 1792x1280 and
down 1280x896 plus 2 shared experts, all per-row INT8; f32 router, softmax top-6 renormalised)
with a residual add between layers, then the 129280 x 1280 BF16 argmax LM head. Each step reads a
fresh seeded f32[1280] ~ N(0,1) hidden state from HBM and writes one token. Weights are seeded
N(0, 0.02) synthetic data generated on the device (no checkpoint is available offline).

The timed region is exactly --steps decode steps, one HIP-graph launch each, bracketed by a device
synchronisation and HIP events on the library stream. Prints one JSON line.
"""
import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
H, I, E, K, SI, VOCAB, LAYERS = 1280, 896, 64, 6, 1792, 129280, 11
DENSE_I = 6848  # layer 0's dense FFN (intermediate_size of DeepSeek-OCR's decoder)
PEAK_HBM_GBS = 8000.0
# HBM bytes per launch of the LM-head kernel, from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of
# this benchmark, scaled by the counters' reading for a 256 MiB device copy (FETCH_SIZE x 2.0,
# WRITE_SIZE x 1.0); profiles/lm_head_argmax_config5_hbm.md holds the runs. Re-measure when the
# kernel changes.
LM_TRAFFIC_BYTES = 331387295
# k_dec_layer<5, 8, 2>, same runs: its own 28.0 MB, the router its verifier blocks read, the input
# and score copies every block reads and its atomic adds (in layer 11 also the next step's router
# partials)
LAYER_TRAFFIC_BYTES = 32621834
LM_CERT_TRAFFIC_BYTES = 170807173  # the bounded head, k_lm_q8_argmax<5, 8>, same method


def product():
    name = "ds_ocr_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "ds-ocr_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def make_layer(dev, seed, gu, dn, rf, rb):
    L = dev.load()
    h = L.ds_hip_layer_create(H, I, E, K, SI)
    if not h:
        raise RuntimeError(L.ds_hip_last_error().decode())
    base = seed * 1000
    for e in range(E):
        dev.check(L.ds_hip_fill_normal_bf16(gu.ptr, 2 * I * H, base + 10 + 2 * e, 0.02), "fill")
        dev.check(L.ds_hip_fill_normal_bf16(dn.ptr, H * I, base + 11 + 2 * e, 0.02), "fill")
        dev.check(L.ds_hip_layer_quantize_expert(h, e, gu.ptr, dn.ptr), "quantize")
    dev.check(L.ds_hip_fill_normal_bf16(gu.ptr, 2 * SI * H, base + 900, 0.02), "fill")
    dev.check(L.ds_hip_fill_normal_bf16(dn.ptr, H * SI, base + 901, 0.02), "fill")
    dev.check(L.ds_hip_layer_quantize_expert(h, -1, gu.ptr, dn.ptr), "quantize")
    dev.check(L.ds_hip_fill_normal_f32(rf.ptr, E * H, base + 1, 0.0, 0.02), "fill")
    dev.check(L.ds_hip_fill_normal_bf16(rb.ptr, E * H, base + 1, 0.02), "fill")
    dev.check(L.ds_hip_layer_set_router_dev(h, rf.ptr, rb.ptr), "router")
    dev.check(L.ds_hip_sync(), "sync")
    return h


def make_dense(dev):
    """DeepSeek-OCR's layer-0 dense FFN (gate/up 6848x1280, down 1280x6848, bf16) with seeded
    N(0, 0.02) weights, rounded to bf16 to nearest even."""
    L = dev.load()
    rng = np.random.default_rng(606)

    def bf16(n):
        u = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)).view(np.uint32)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    g, u, d = bf16(DENSE_I * H), bf16(DENSE_I * H), bf16(H * DENSE_I)
    D = L.ds_hip_dense_create(H, DENSE_I, g.ctypes.data, u.ctypes.data, d.ctypes.data)
    if not D:
        raise RuntimeError(L.ds_hip_last_error().decode())
    return D


def make_attention(dev, n, kv, max_seq):
    """n decoder attention blocks (DeepSeek-OCR: 10 heads x 128, seeded N(0, 0.02) bf16 projections,
    unit norms) with kv seeded cached positions each."""
    L = dev.load()
    rng = np.random.default_rng(909)
    qd = 10 * 128

    def bf16(m):
        u = (rng.standard_normal(m, dtype=np.float32) * np.float32(0.02)).view(np.uint32)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    ones = np.ones(H, np.float32)
    out = []
    for _ in range(n):
        w = [bf16(qd * H) for _ in range(4)]
        A = L.ds_hip_attn_create(H, 10, 128, max_seq, 1e-6, 10000.0, *[a.ctypes.data for a in w], ones.ctypes.data,
                                 ones.ctypes.data, None, None)
        if not A:
            raise RuntimeError(L.ds_hip_last_error().decode())
        if kv:
            k = (rng.standard_normal(kv * qd, dtype=np.float32) * np.float32(0.3))
            v = rng.standard_normal(kv * qd, dtype=np.float32)
            dev.check(L.ds_hip_attn_load_kv(A, k.ctypes.data, v.ctypes.data, kv, qd), "kv")
        out.append(A)
    return out


def host_layers(dev, handles, rf_host, rb_host):
    """Copies the device layers' INT8 blocks to the host (for the reference CPU baseline)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import bindings as B
    L = dev.load()
    out = []
    for li, h in enumerate(handles):
        gus, dns = [], []
        for e in list(range(E)) + [-1]:
            ii = SI if e < 0 else I
            gq = np.empty((2 * ii, H), np.int8)
            gs = np.empty(2 * ii, np.float32)
            go = np.empty(2 * ii, np.float32)
            dq = np.empty((H, ii), np.int8)
            ds = np.empty(H, np.float32)
            do = np.empty(H, np.float32)
            dev.check(L.ds_hip_layer_export_expert(h, e, gq.ctypes.data, gs.ctypes.data, go.ctypes.data,
                                                   dq.ctypes.data, ds.ctypes.data, do.ctypes.data), "export")
            gus.append(B.QBlock(gq, gs, go))
            dns.append(B.QBlock(dq, ds, do))
        out.append(B.MoELayer(H, I, E, K, SI, rf_host[li], rb_host[li], gus[:E], dns[:E], gus[E], dns[E]))
    return out


def cpu_model():
    for line in open("/proc/cpuinfo"):
        if line.startswith("model name"):
            return line.split(":", 1)[1].strip()
    return "unknown"


def ref_variant():
    flags = open("/proc/cpuinfo").read()
    return "v4" if (" avx512f " in flags and " avx512bw " in flags) else "v3"


def cpu_baseline(lays, lm_w, xs_host, gpu_tokens, route, budget_s, dropin=None):
    """The reference CPU path (ds-ocr's own C, oracle/_ref) on this host: moe_forward's INT8 branch
    for 11 layers + ds_argmax_matvec_bf16 per step. Rows: the reference's own thread count
    (min(cores, 16): ds_kernels.c:123, :518-519 clamp it) and 1 thread in the bench's routing, and
    the reference thread count in DECODE routing (moe_forward's own router) beside the drop-in leg;
    each row runs a bounded sample of the same steps (about budget_s of CPU time)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import bindings as B
    variant = ref_variant()
    R = B.ref(variant)
    if R is None:
        return None
    bufs = [lay.ref_layer(variant) for lay in lays]
    arr = C.create_string_buffer(len(bufs) * R.ref_layer_sizeof())
    for i, b in enumerate(bufs):
        C.memmove(C.addressof(arr) + i * R.ref_layer_sizeof(), b, R.ref_layer_sizeof())
    ncpu = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else ncpu
    clamp = min(16, affinity)
    rows = []
    plan = [(clamp, route)] + ([(1, route)] if clamp > 1 else [])
    if dropin is not None:
        plan.append((clamp, 0))
    for threads, rt in plan:
        R.ds_set_threads(threads)
        toks = np.zeros(len(xs_host), np.int32)
        t1 = R.ref_decode_steps(C.addressof(arr), LAYERS, lm_w, VOCAB, xs_host, 1, rt, toks)
        n = int(max(1, min(len(xs_host), budget_s / max(t1, 1e-6))))
        secs = R.ref_decode_steps(C.addressof(arr), LAYERS, lm_w, VOCAB, xs_host, n, rt, toks)
        row = {"threads": threads, "route": "cfg" if rt == 1 else "decode", "value": round(n / secs, 3),
               "unit": "tok/s", "ms_per_step": round(1000 * secs / n, 3), "steps": n}
        if rt == route:
            row["tokens_equal_to_gpu"] = int(np.sum(toks[:n] == gpu_tokens[:n]))
        if dropin is not None and rt == 0:
            m = min(n, len(dropin["tokens"]))
            dropin["tokens_equal_to_reference_decode_route"] = f"{int(np.sum(toks[:m] == dropin['tokens'][:m]))}/{m}"
        rows.append(row)
    main = rows[0]
    return {"value": main["value"], "unit": "tok/s", "cores": main["threads"], "kind": "reference",
            "sample": f"{main['steps']} decode steps of the same 11-layer + LM-head workload (the timed region's "
                      f"first {main['steps']} inputs, same weights exported from the device), reference ds-ocr C "
                      f"path built -O3 -march=x86-64-{variant}, {main['threads']} threads (the reference clamps "
                      f"to 16) on '{cpu_model()}'; tokens equal to the GPU's on "
                      f"{main['tokens_equal_to_gpu']}/{main['steps']} steps",
            "ms_per_step": main["ms_per_step"], "rows": rows,
            "host": {"cpu": cpu_model(), "logical_cpus": ncpu, "affinity_cpus": affinity},
            "unclamped_row": ("not run: the reference's thread pool clamps to 16 threads (ds_kernels.c:123, "
                              f":518-519) and this process may use {affinity} CPUs" if affinity > 16 else
                              f"equal to the clamped row: this process may use {affinity} CPUs")}


class DropinLayer(C.Structure):
    """dropin_layer_t of ds-ocr_amd/examples/moe_forward_dropin.c."""
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
                ("shared_inter", C.c_int), ("router_bf16", C.c_void_p), ("gate_up", C.c_void_p),
                ("down", C.c_void_p), ("shared_gate_up", C.c_void_p), ("shared_down", C.c_void_p)]


def dropin_leg(dev, lays, lm_w, xs_host, n_steps):
    """The per-function drop-in path: the reference's decode step (moe_forward's calls for 11 layers,
    then ds_argmax_matvec_bf16) through the C API with host pointers, as an unchanged reference
    caller runs it (ds-ocr_amd/examples/moe_forward_dropin.c); weights registered once first."""
    ex = C.CDLL(os.path.join(ROOT, "ds-ocr_amd", "examples", "libdropin_example.so"))
    ex.dropin_register.restype = C.c_int
    ex.dropin_register.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int]
    ex.dropin_decode_steps.restype = C.c_double
    ex.dropin_decode_steps.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]
    ex.dropin_call_times.restype = None
    ex.dropin_call_times.argtypes = [C.c_void_p, C.c_void_p]
    keep = []
    arr = (DropinLayer * len(lays))()
    for l, lay in enumerate(lays):
        gu = (dev.Int4Block * lay.n_experts)(*[dev.block_from_arrays(b.q, b.scale, b.offset) for b in lay.gu])
        dn = (dev.Int4Block * lay.n_experts)(*[dev.block_from_arrays(b.q, b.scale, b.offset) for b in lay.dn])
        sgu = dev.block_from_arrays(lay.sgu.q, lay.sgu.scale, lay.sgu.offset)
        sdn = dev.block_from_arrays(lay.sdn.q, lay.sdn.scale, lay.sdn.offset)
        keep += [gu, dn, sgu, sdn]
        arr[l] = DropinLayer(lay.hidden, lay.inter, lay.n_experts, lay.top_k, lay.shared_inter,
                             lay.router_bf16.ctypes.data, C.addressof(gu), C.addressof(dn), C.addressof(sgu),
                             C.addressof(sdn))
    t0 = time.perf_counter()
    if ex.dropin_register(C.addressof(arr), len(lays), lm_w.ctypes.data, VOCAB):
        raise RuntimeError("drop-in registration: " + dev.load().ds_hip_last_error().decode())
    reg_s = time.perf_counter() - t0
    n = min(n_steps, len(xs_host))
    toks = np.zeros(len(xs_host), np.int32)
    ex.dropin_decode_steps(C.addressof(arr), len(lays), lm_w.ctypes.data, VOCAB, xs_host.ctypes.data, 1,
                           toks.ctypes.data)  # warm-up step
    secs = ex.dropin_decode_steps(C.addressof(arr), len(lays), lm_w.ctypes.data, VOCAB, xs_host.ctypes.data, n,
                                  toks.ctypes.data)
    if secs <= 0:
        raise RuntimeError("drop-in leg failed")
    ks, kc = (C.c_double * 6)(), (C.c_long * 6)()
    ex.dropin_call_times(ks, kc)
    kinds = ["ds_moe_router_bf16", "ds_expert_forward_fused_int4 (routed)", "ds_expert_combine",
             "ds_expert_forward_fused_int4 (shared)", "ds_vec_add", "ds_argmax_matvec_bf16"]
    per_call = {kinds[k]: {"calls_per_step": round(kc[k] / n, 2), "us_per_call": round(1e6 * ks[k] / max(kc[k], 1), 2),
                           "us_per_step": round(1e6 * ks[k] / n, 1)} for k in range(6)}
    return {"value": round(n / secs, 3), "unit": "tok/s", "ms_per_step": round(1000 * secs / n, 3), "steps": n,
            "route": "decode (moe_forward's bf16 router, host softmax/top-k as the reference caller does it)",
            "register_s": round(reg_s, 2), "tokens": toks[:n], "per_call": per_call,
            "calls_per_step": LAYERS * (1 + K + 1 + 1 + 2) + 1,
            "method": "host wall clock around n steps of ds-ocr_amd/examples/moe_forward_dropin.c: per layer "
                      "ds_moe_router_bf16, 6 x ds_expert_forward_fused_int4, ds_expert_combine, the shared "
                      "expert, 2 x ds_vec_add; then ds_argmax_matvec_bf16; every call synchronous with host "
                      "activations (the drop-in boundary)"}


def fast_expf_np(x):
    """ds_fast_expf (ds_kernels.h:296-302) vectorised: Schraudolph's bit trick with GCC's fused
    12102203*x + 1064866805, saturating below -88 and above 88."""
    x = np.asarray(x, np.float32)
    v = (np.float64(12102203.0) * x.astype(np.float64) + 1064866805.0).astype(np.float32)  # one rounding: fused
    out = v.astype(np.int64).astype(np.uint32).view(np.float32)
    out = np.where(x < -88.0, np.float32(0.0), out)
    return np.where(x > 88.0, np.float32(1e38), out).astype(np.float32)


def prefill_cpu_baseline(lay, X, reps, budget_s):
    """The reference's prefill MoE block (ds_moe_decoder.c:629-809) on the host: router sgemm, the
    fast-exp softmax and top-k per token, the shared expert and every routed expert's gathered
    tokens as sgemm calls (gate, up, down), scatter-add of the weighted outputs, residual. The
    sgemms are OpenBLAS's (numpy's bundled OpenBLAS, the library the reference links for cblas_sgemm).
    Weights are f32 copies made once (the reference's cached f32 views, ds_kernels.c:751-759); they
    are the INT8 codes dequantized, the same values the GPU multiplies."""
    H_, I_, E_, K_ = lay.hidden, lay.inter, lay.n_experts, lay.top_k

    def deq(b):
        return (b.scale[:, None] * (b.q.astype(np.float32) + np.float32(128.0)) + b.offset[:, None]).astype(np.float32)

    gw = [deq(b) for b in lay.gu]
    dw = [deq(b) for b in lay.dn]
    sg, sd = deq(lay.sgu), deq(lay.sdn)
    SI_ = lay.shared_inter
    wr = (lay.router_bf16.astype(np.uint32) << 16).view(np.float32).reshape(E_, H_)

    def silu_mul(g, u):
        return (g / (np.float32(1.0) + fast_expf_np(-g))) * u

    def one_call():
        T_ = X.shape[0]
        sc = X @ wr.T
        p = fast_expf_np(sc - sc.max(axis=1, keepdims=True))
        p = p * (np.float32(1.0) / p.sum(axis=1, dtype=np.float32, keepdims=True))
        idx = np.argsort(-p, axis=1, kind="stable")[:, :K_]
        wts = np.take_along_axis(p, idx, axis=1)
        shared = silu_mul(X @ sg[:SI_].T, X @ sg[SI_:].T) @ sd.T
        routed = np.zeros((T_, H_), np.float32)
        for e in range(E_):
            tok, slot = np.nonzero(idx == e)
            if tok.size == 0:
                continue
            xe = X[tok]
            out = silu_mul(xe @ gw[e][:I_].T, xe @ gw[e][I_:].T) @ dw[e].T
            routed[tok] += wts[tok, slot][:, None] * out
        return X + (routed + shared), idx

    out, idx = one_call()  # warm-up
    t1 = time.perf_counter()
    one_call()
    t_one = time.perf_counter() - t1
    n = int(max(1, min(reps, budget_s / max(t_one, 1e-6))))
    times = []
    for _ in range(n):
        t0 = time.perf_counter()
        one_call()
        times.append(time.perf_counter() - t0)
    try:
        from threadpoolctl import threadpool_info
        blas_threads = [i.get("num_threads") for i in threadpool_info() if i.get("user_api") == "blas"]
    except Exception:  # report, never hide
        blas_threads = []
    return {"median_ms": round(1e3 * float(np.median(times)), 3), "p10_ms": round(1e3 * float(np.percentile(times, 10)), 3),
            "p90_ms": round(1e3 * float(np.percentile(times, 90)), 3), "calls": n,
            "threads": blas_threads[0] if blas_threads else None,
            "kind": "port: the reference's prefill block in numpy with OpenBLAS 0.3 sgemm (numpy's bundled OpenBLAS)",
            "routing": "bf16 router widened, fast-exp softmax over 64, top-6 (the reference prefill's own routing)",
            "note": "weights pre-converted to f32 once (the reference's cached f32 views); a call without the "
                    "cache also converts every expert's weights"}, out, idx


def pct(v, q):
    return round(float(np.percentile(np.asarray(v, np.float64), q)), 5)


def bench_plan(steps, warmup, each, span, profile):
    """The main stack's step-running calls, as phases separated by resets: (call, steps) in order.
    Returns the input rows / token slots the stack needs and the phases."""
    phases = [[("run", warmup), ("time", steps)], [("each", each)], [("profile", profile)], [("span", span)]]
    rows = max(1, max(sum(n for _, n in ph) for ph in phases))
    return rows, phases


def decoder_plan(n_warm, n_timed):
    phases = [[("run", n_warm), ("time", n_timed)]]
    return n_warm + n_timed, phases


def check_plan(L, rows, stride, n_tokens, kv_room, phases):
    """Checks every phase of a plan against the stack's capacity rule before anything runs."""
    cap = L.ds_hip_stack_capacity_for(rows, stride, n_tokens, kv_room)
    if cap < 0:
        raise ValueError(f"invalid stack buffers: rows {rows}, stride {stride}, tokens {n_tokens}")
    for ph in phases:
        done = 0
        for call, n in ph:
            if not L.ds_hip_steps_fit(cap, done, n):
                raise ValueError(f"plan {ph}: {call} of {n} steps after {done} passes the capacity {cap}")
            done += n
    return cap


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=226)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--route", choices=["cfg", "decode"], default="cfg")
    ap.add_argument("--dist-steps", type=int, default=200,
                    help="graph launches timed one by one for the median and p10/p90 (at least 100)")
    ap.add_argument("--span-steps", type=int, default=100,
                    help="eager steps whose MoE-layer span gives the layer kernel's average duration")
    ap.add_argument("--profile-steps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-dropin", action="store_true", help="skip the per-function drop-in leg")
    ap.add_argument("--dropin-steps", type=int, default=20)
    ap.add_argument("--prefill-tokens", type=int, default=662, help="config-3 prefill measurement (0: skip)")
    ap.add_argument("--prefill-reps", type=int, default=100)
    ap.add_argument("--dense-layer", action="store_true",
                    help="prepend DeepSeek-OCR's layer-0 dense SwiGLU FFN (1280x6848 bf16) to every step")
    ap.add_argument("--decoder-step", type=int, default=-1, metavar="KV",
                    help=">= 0: whole decoder steps (attention 10x128 + MLP per layer, the dense layer 0, final "
                         "norm) after KV cached positions")
    ap.add_argument("--decoder-kv", type=int, default=1000,
                    help="also time whole decoder steps (attention + MLP per layer, final norm, head) after this "
                         "many cached positions, as the line's 'decoder_step' entry (-1: skip)")
    ap.add_argument("--repeat-penalty", type=float, default=1.0,
                    help="> 1: the reference's repetition penalty after each argmax, over the run's tokens")
    ap.add_argument("--no-repeat-ngram", type=int, default=0, help="> 0: the reference's n-gram ban")
    ap.add_argument("--lm-head", choices=["bounded", "one-pass"], default="bounded",
                    help="LM-head argmax: an int8 copy with exact bounds, then each block's candidate rows in bf16 "
                         "(the same tokens), or the one-pass bf16 kernel")
    ap.add_argument("--graph-steps", type=int, default=8,
                    help="decode steps per graph launch in the timed runs (the same results for every value)")
    ap.add_argument("--layer-kernels", type=int, choices=[1, 2], default=1,
                    help="MoE layer kernels: 1 (down split over intermediate units, per-XCD output copies) or 2 "
                         "(gate_up, then down with the combine in top-k order)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="run one device-to-device copy of this many MiB first (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (sharding the decode "
                                   "path over several GPUs is not implemented)"}))
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        sys.exit("--steps must be >= 1 and --warmup >= 0")
    dev = product()
    L = dev.load()
    route = dev.ROUTE_CFG if args.route == "cfg" else dev.ROUTE_DECODE
    full = args.decoder_step >= 0
    n_each = max(100, args.dist_steps)
    n_span = max(10, args.span_steps)
    rows, phases = bench_plan(args.steps, args.warmup, n_each, n_span, args.profile_steps)
    kv_room = rows + 1 if full else -1
    check_plan(L, rows, H, rows, kv_room, phases)
    n_dec_warm, n_dec = 5, 40
    dec_rows, dec_phases = decoder_plan(n_dec_warm, n_dec)
    if args.decoder_kv >= 0 and not full:
        check_plan(L, dec_rows, H, dec_rows, dec_rows + 1, dec_phases)
    dev.check(L.ds_hip_init(), "init")

    gu = dev.DeviceBuffer(2 * SI * H * 2)
    dn = dev.DeviceBuffer(H * SI * 2)
    rfs = [dev.DeviceBuffer(E * H * 4) for _ in range(LAYERS)]
    rbs = [dev.DeviceBuffer(E * H * 2) for _ in range(LAYERS)]
    handles = [make_layer(dev, 100 + l, gu, dn, rfs[l], rbs[l]) for l in range(LAYERS)]
    gu.close()
    dn.close()
    lm = dev.DeviceBuffer(VOCAB * H * 2)
    dev.check(L.ds_hip_fill_normal_bf16(lm.ptr, VOCAB * H, 4242, 0.02), "fill")
    if args.copy_calibration_mb > 0:
        nb = args.copy_calibration_mb << 20
        src, dst = dev.DeviceBuffer(nb), dev.DeviceBuffer(nb)
        dev.check(L.ds_hip_memcpy_d2d(dst.ptr, src.ptr, nb), "calibration copy")
        dev.check(L.ds_hip_sync(), "sync")
        src.close()
        dst.close()
    xs = dev.DeviceBuffer(rows * H * 4)
    dev.check(L.ds_hip_fill_normal_f32(xs.ptr, rows * H, 777, 0.0, 1.0), "fill")
    toks = dev.DeviceBuffer(rows * 4)
    arr = (C.c_void_p * LAYERS)(*handles)
    S = L.ds_hip_stack_create(arr, LAYERS, lm.ptr, VOCAB, route)
    if not S:
        raise RuntimeError(L.ds_hip_last_error().decode())
    sampling = args.repeat_penalty > 1.0 or args.no_repeat_ngram > 0
    if sampling:
        dev.check(L.ds_hip_stack_set_sampling(S, args.repeat_penalty, args.no_repeat_ngram, rows), "sampling")
    dense = make_dense(dev) if (args.dense_layer or full) else None
    if dense:
        dev.check(L.ds_hip_stack_set_dense(S, dense), "set dense")
    attns = []
    if full:
        attns = make_attention(dev, LAYERS + 1, args.decoder_step, args.decoder_step + kv_room)
        fnorm = np.ones(H, np.float32)
        arr_a = (C.c_void_p * len(attns))(*attns)
        dev.check(L.ds_hip_stack_set_attention(S, arr_a, len(attns), fnorm.ctypes.data, 1e-6, args.decoder_step, 0),
                  "set attention")
    dev.check(L.ds_hip_stack_set_layer_kernels(S, 1 if args.layer_kernels == 1 else 0), "layer kernels")
    dev.check(L.ds_hip_stack_set_graph_steps(S, args.graph_steps), "graph steps")
    if args.lm_head == "one-pass":
        dev.check(L.ds_hip_stack_set_lm_certified(S, 0), "one-pass LM head")
    cert = L.ds_hip_stack_lm_certified(S) == 1
    dev.check(L.ds_hip_stack_bind(S, xs.ptr, H, rows, toks.ptr, rows), "bind")
    if L.ds_hip_stack_capacity(S) < rows:
        raise RuntimeError(f"stack capacity {L.ds_hip_stack_capacity(S)} < planned {rows}")
    bytes_per_step = L.ds_hip_stack_bytes_per_step(S)
    layer_kernels = L.ds_hip_stack_layer_kernels(S)
    nk = L.ds_hip_stack_kernel_count(S)
    names = [L.ds_hip_stack_kernel_name(S, i).decode() for i in range(nk)]

    # warmup, then exactly --steps timed steps (graph launches) between synchronisations
    dev.check(L.ds_hip_stack_run(S, args.warmup), "warmup")
    dev.check(L.ds_hip_sync(), "sync")
    rstat = (C.c_ulonglong * 3)()
    dev.check(L.ds_hip_route_stats(rstat, 1), "route counters")
    ms = C.c_float(0)
    t0 = time.perf_counter()
    dev.check(L.ds_hip_time_stack(S, args.steps, C.byref(ms)), "timed steps")
    dev.check(L.ds_hip_sync(), "sync")
    wall = time.perf_counter() - t0
    gpu_tokens = toks.to_array(np.int32)[args.warmup:args.warmup + args.steps].copy()
    ms_per_step = ms.value / args.steps
    dev.check(L.ds_hip_route_stats(rstat, 1), "route counters")
    n_route = int(rstat[0])
    route_cert = {"routings": n_route, "recomputed": int(rstat[1]), "corrected": int(rstat[2]),
                  "fallback_rate": round(rstat[1] / n_route, 5) if n_route else None,
                  "correction_rate": round(rstat[2] / n_route, 5) if n_route else None,
                  "note": "the timed steps' CFG expert selections, every one certified against ds_linear's order: "
                          "recomputed = the intervals did not separate the ranks, so the open experts' scores were "
                          "recomputed in that order; corrected = the one-kernel layer's speculative selection "
                          "differed from the certified one and its output was corrected (ms_per_step includes all "
                          "of it)"} if route == dev.ROUTE_CFG else None

    # the step-time distribution: n_each graph launches with an event between consecutive ones
    dev.check(L.ds_hip_stack_reset(S), "reset")
    dev.check(L.ds_hip_stack_run(S, 0), "run")
    each = np.zeros(n_each, np.float32)
    dev.check(L.ds_hip_time_stack_each(S, n_each, each), "per-step timing")
    rerun = toks.to_array(np.int32)
    lo, hi = args.warmup, min(args.warmup + args.steps, n_each)
    rerun_equal = int(np.sum(rerun[lo:hi] == gpu_tokens[:max(0, hi - lo)])) if hi > lo else 0

    # per-kernel durations (eager launches with HIP events around every kernel)
    dev.check(L.ds_hip_stack_reset(S), "reset")
    per = np.zeros(nk, np.float32)
    dev.check(L.ds_hip_profile_stack(S, args.profile_steps, per), "profile")
    kinds = {}
    for k, v in zip(names, per):
        kinds.setdefault(k, []).append(float(v))
    kernel_ms = {k: {"avg_ms": round(float(np.mean(v)), 5), "launches_per_step": len(v),
                     "ms_per_step": round(float(np.sum(v)), 5)} for k, v in kinds.items()}

    # the MoE layers' span inside real eager steps: events before the first and after the last layer
    # kernel only, so the span / 11 is the layer kernel's average launch duration on real inputs, over
    # 11 distinct layers' weights (308 MB per step, more than the 256 MB MALL)
    moe = [i for i, n in enumerate(names)
           if n in ("layer", "gate_up", "down") or (n == "scores" and route == dev.ROUTE_DECODE)]
    dev.check(L.ds_hip_stack_reset(S), "reset")
    span = np.zeros(n_span, np.float32)
    dev.check(L.ds_hip_time_stack_span(S, n_span, moe[0], moe[-1] + 1, span), "layer span timing")
    # the head's bytes per step: the bf16 rows, or (bounded) the int8 codes and 12 bytes of
    # constants per row (the few candidate rows read again in bf16 are not counted)
    lm_bytes = VOCAB * (H + 12) if cert else VOCAB * H * 2
    dense_bytes = 3 * H * DENSE_I * 2 if dense else 0
    attn_bytes = 0
    layer_bytes = (bytes_per_step - lm_bytes - dense_bytes - attn_bytes) // LAYERS
    layer_ms = float(np.median(span)) / LAYERS
    layer_gbs = layer_bytes / (layer_ms * 1e-3) / 1e9
    layer_kernel = ("k_dec_layer (one kernel per MoE layer: k_dec_layer<5, 1, 40> for the first, k_dec_layer<5, 8, 2> "
                    "for the other 10)" if layer_kernels == 1 else "k_dec_gate_up<5> + k_dec_down<8> (two kernels per "
                                                                   "MoE layer)")
    if route == dev.ROUTE_DECODE:
        layer_kernel += " with its k_dec_scores_bf16 kernel"
    roofline = {"kernel": layer_kernel, "bound": "hbm", "achieved": round(layer_gbs, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(layer_gbs / PEAK_HBM_GBS, 4),
                "traffic": LAYER_TRAFFIC_BYTES if (layer_kernels == 1 and route == dev.ROUTE_CFG and not full) else None,
                "bytes_per_launch": int(layer_bytes), "launches_per_step": LAYERS,
                "avg_ms": round(layer_ms, 5), "p10_ms": round(pct(span, 10) / LAYERS, 5),
                "p90_ms": round(pct(span, 90) / LAYERS, 5),
                "avg_ms_method": f"median over {n_span} eager steps of the span from the first to the last MoE-layer "
                                 "kernel (HIP events on the library stream, none between the layers), divided by "
                                 f"{LAYERS}: real inputs and 11 distinct layers' weights; includes the kernel "
                                 "boundaries between the layers",
                "why_this_kernel": "the MoE layers take the largest share of the step (11 launches), ahead of the "
                                   "LM head (1 launch)"}
    # the LM-head kernel alone, 50 launches back to back on the last step's hidden state
    lm_t = C.c_float(0)
    dev.check(L.ds_hip_time_lm_head(S, 50, C.byref(lm_t)), "lm head timing")
    lm_ms = lm_t.value
    lm_gbs = lm_bytes / (lm_ms * 1e-3) / 1e9
    # achievable HBM read rate on this box: a plain streaming read of the same 331 MB
    rd_t = C.c_float(0)
    dev.check(L.ds_hip_time_stream_read(lm.ptr, lm_bytes, 50, C.byref(rd_t)), "stream read timing")
    read_gbs = lm_bytes / (rd_t.value * 1e-3) / 1e9
    lm_kernel = ("k_lm_q8_argmax<5, 0> (LM-head argmax, 1 launch per step: the int8 copy of the head with a bound "
                 "on every row's exact logit, then each block's candidate rows in the reference's bf16 order; the "
                 "step runs k_lm_q8_argmax<5, 8> on the layer copies)" if cert else
                 "k_dec_lm_argmax<1, 8> (LM-head argmax, 1 launch per step)")
    roofline_lm = {"kernel": lm_kernel, "bound": "hbm",
                   "achieved": round(lm_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                   "frac": round(lm_gbs / PEAK_HBM_GBS, 4), "traffic": LM_CERT_TRAFFIC_BYTES if cert else LM_TRAFFIC_BYTES,
                   "bytes_per_launch": lm_bytes, "reference_bytes_per_launch": VOCAB * H * 2, "avg_ms": round(lm_ms, 5),
                   "avg_ms_method": "50 back-to-back launches between HIP events on the library stream, on the "
                                    "last step's hidden state",
                   "stream_read_gbs": round(read_gbs, 1), "frac_of_stream_read": round(lm_gbs / read_gbs, 4),
                   "stream_read_note": "a plain nontemporal streaming read of the same bytes, timed the same way: "
                                       "the achievable HBM read rate on this box"}
    step_gbs = bytes_per_step / (ms_per_step * 1e-3) / 1e9

    # prefill (config 3): 662 seeded tokens through one config-2 layer (the first decode layer)
    prefill = None
    pf_host = None
    if args.prefill_tokens > 0:
        T = args.prefill_tokens
        xp = dev.DeviceBuffer(T * H * 4)
        dev.check(L.ds_hip_fill_normal_f32(xp.ptr, T * H, 662, 0.0, 1.0), "fill")
        op = dev.DeviceBuffer(T * H * 4)
        pt = C.c_float(0)
        dev.check(L.ds_hip_time_prefill(handles[0], op.ptr, xp.ptr, T, route, args.prefill_reps, C.byref(pt)),
                  "prefill timing")
        us = pt.value * 1e3
        # algorithmic work: K routed + shared experts per token (2 flops per weight element) and the router
        flops = T * (K * 2 * (2 * I * H + H * I) + 2 * (2 * SI * H + H * SI) + 2 * E * H)
        wbytes = E * (2 * I * H + 2 * I * 8 + H * I + H * 8) + 2 * SI * H + 2 * SI * 8 + H * SI + H * 8
        if not args.no_cpu:  # the GPU's output in the reference prefill's own routing, for the CPU leg
            idx_d = dev.DeviceBuffer(T * K * 4)
            dev.check(L.ds_hip_layer_prefill(handles[0], op.ptr, xp.ptr, T, dev.ROUTE_DECODE, 1, idx_d.ptr, None),
                      "prefill")
            pf_host = (xp.to_array(np.float32).reshape(T, H), op.to_array(np.float32).reshape(T, H),
                       idx_d.to_array(np.int32).reshape(T, K))
            idx_d.close()
        prefill = {"config": "config 3: 662 tokens x 1280 through one config-2 layer", "tokens": T,
                   "us": round(us, 2), "tok_per_s": round(T / (us * 1e-6), 1),
                   "algorithmic_tflops": round(flops / (us * 1e-6) / 1e12, 2),
                   "mfma_frac_of_int8_peak": round(2 * flops / (us * 1e-6) / 5.0e15, 4),
                   "weight_bytes": wbytes, "weight_gbs": round(wbytes / (us * 1e-6) / 1e9, 1),
                   "hbm_frac": round(wbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                   "us_method": f"{args.prefill_reps} back-to-back calls (one graph launch each) between HIP events",
                   "note": "the GEMMs run on the int8 MFMA (5.0 POP/s dense) with each activation as two "
                           "8-bit limbs: executed work is 2x the algorithmic flops, and the fraction counts it"}
        xp.close()
        op.close()

    # configs 1 and 2 on their own (BASELINE's GB/s rows): one expert through the per-function
    # kernel, one MoE layer through ds_hip_layer_forward, inputs and outputs in device memory
    singles = None
    if not full:
        gq, gs, go = np.empty((2 * I, H), np.int8), np.empty(2 * I, np.float32), np.empty(2 * I, np.float32)
        dq, ds_, do = np.empty((H, I), np.int8), np.empty(H, np.float32), np.empty(H, np.float32)
        dev.check(L.ds_hip_layer_export_expert(handles[0], 0, gq.ctypes.data, gs.ctypes.data, go.ctypes.data,
                                               dq.ctypes.data, ds_.ctypes.data, do.ctypes.data), "export")
        gb, db = dev.block_from_arrays(gq, gs, go), dev.block_from_arrays(dq, ds_, do)
        x1 = np.random.default_rng(1).standard_normal(H).astype(np.float32)
        te = C.c_float(0)
        dev.check(L.ds_hip_time_expert(C.byref(gb), C.byref(db), H, I, x1.ctypes.data, 200, C.byref(te)),
                  "expert timing")
        e_bytes = 2 * I * H + 2 * I * 8 + H * I + H * 8
        xl = dev.DeviceBuffer(H * 4)
        dev.check(L.ds_hip_fill_normal_f32(xl.ptr, H, 4711, 0.0, 1.0), "fill")
        ol = dev.DeviceBuffer(H * 4)
        tl = C.c_float(0)
        dev.check(L.ds_hip_time_layer(handles[0], ol.ptr, xl.ptr, route, 200, C.byref(tl)), "layer timing")
        l_bytes = K * e_bytes + (2 * SI * H + 2 * SI * 8 + H * SI + H * 8) + E * H * 4
        singles = {
            "config1_expert": {"bytes": e_bytes, "us": round(te.value * 1e3, 2),
                               "gbs": round(e_bytes / (te.value * 1e-3) / 1e9, 1),
                               "frac": round(e_bytes / (te.value * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                               "kernel": "k_expert_exact (ds_expert_forward_fused_int4's one launch: every row "
                                         "in the reference's sequential order, bit-identical)",
                               "method": "200 back-to-back launches between HIP events, x and y in device memory"},
            "config2_layer": {"bytes": l_bytes, "us": round(tl.value * 1e3, 2),
                              "gbs": round(l_bytes / (tl.value * 1e-3) / 1e9, 1),
                              "frac": round(l_bytes / (tl.value * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                              "kernel": "ds_hip_layer_forward: k_dec_gate_up + k_dec_down (the two-kernel layer, "
                                        "certified CFG routing), one layer on its own",
                              "method": "200 back-to-back calls between HIP events; in the stack the one-kernel "
                                        "layer's time is roofline.avg_ms"}}
        xl.close()
        ol.close()

    # whole decoder steps (12 layers with their attention halves after kv cached positions), with
    # their own input rows and token slots
    decoder = None
    if args.decoder_kv >= 0 and not full:
        kv = args.decoder_kv
        dense2 = make_dense(dev)
        attns2 = make_attention(dev, LAYERS + 1, kv, kv + dec_rows + 1)
        arr2 = (C.c_void_p * LAYERS)(*handles)
        S2 = L.ds_hip_stack_create(arr2, LAYERS, lm.ptr, VOCAB, route)
        if not S2:
            raise RuntimeError(L.ds_hip_last_error().decode())
        dev.check(L.ds_hip_stack_set_dense(S2, dense2), "set dense")
        fnorm = np.ones(H, np.float32)
        arr_a2 = (C.c_void_p * len(attns2))(*attns2)
        dev.check(L.ds_hip_stack_set_attention(S2, arr_a2, len(attns2), fnorm.ctypes.data, 1e-6, kv, 0), "attention")
        xs2 = dev.DeviceBuffer(dec_rows * H * 4)
        dev.check(L.ds_hip_fill_normal_f32(xs2.ptr, dec_rows * H, 778, 0.0, 1.0), "fill")
        toks2 = dev.DeviceBuffer(dec_rows * 4)
        dev.check(L.ds_hip_stack_set_layer_kernels(S2, 1 if args.layer_kernels == 1 else 0), "layer kernels")
        dev.check(L.ds_hip_stack_bind(S2, xs2.ptr, H, dec_rows, toks2.ptr, dec_rows), "bind")
        dev.check(L.ds_hip_stack_run(S2, n_dec_warm), "warmup")
        dev.check(L.ds_hip_sync(), "sync")
        ms2 = C.c_float(0)
        dev.check(L.ds_hip_time_stack(S2, n_dec, C.byref(ms2)), "timed decoder steps")
        step_ms = ms2.value / n_dec
        decoder = {"config": f"12 decoder layers (dense layer 0 + the 11 MoE layers above), each with its attention "
                             f"half (10 heads x 128, f32 KV cache), final RMSNorm, argmax head; tokens at cache "
                             f"positions {kv + n_dec_warm}..{kv + dec_rows - 1} after {kv} seeded cached positions",
                   "steps": n_dec, "ms_per_step": round(step_ms, 5), "tok_per_s": round(1e3 / step_ms, 2),
                   "bytes_per_step_weights": int(L.ds_hip_stack_bytes_per_step(S2)),
                   "note": "bytes exclude the KV reads (about 10 KB per cached position and layer)"}
        L.ds_hip_stack_destroy(S2)
        for A in attns2:
            L.ds_hip_attn_destroy(A)
        L.ds_hip_dense_destroy(dense2)
        toks2.close()
        xs2.close()

    xs_host = xs.to_array(np.float32).reshape(rows, H)[args.warmup:args.warmup + args.steps].copy()
    cpu = None
    dropin = None
    if not args.no_cpu and not dense and not sampling and not full:  # the reference CPU leg: MoE layers + argmax head
        try:
            lays = host_layers(dev, handles, [rf.to_array(np.float32) for rf in rfs],
                               [rb.to_array(np.uint16) for rb in rbs])
            lm_w = lm.to_array(np.uint16)
            if not args.no_dropin:
                try:
                    dropin = dropin_leg(dev, lays, lm_w, xs_host, args.dropin_steps)
                except Exception as exc:  # report, never hide
                    dropin = {"error": repr(exc)}
            cpu = cpu_baseline(lays, lm_w, xs_host, gpu_tokens, route, args.cpu_seconds,
                               dropin if dropin and "tokens" in dropin else None)
            if dropin and "tokens" in dropin:
                dropin.pop("tokens")
                ref_dec = [r for r in cpu["rows"] if r["route"] == "decode"] if cpu else []
                if ref_dec:
                    dropin["vs_cpu_baseline_decode_route"] = round(dropin["value"] / ref_dec[0]["value"], 3)
            if prefill is not None and pf_host is not None:
                try:
                    pcpu, pout, pidx = prefill_cpu_baseline(lays[0], pf_host[0], 20, args.cpu_seconds)
                    d = np.abs(pout.astype(np.float64) - pf_host[1]).max() / np.abs(pf_host[1]).max()
                    pcpu["gpu_vs_cpu"] = {"max_abs_err_over_max": float(f"{d:.3e}"),
                                          "routing_equal_tokens": f"{int(np.sum(np.all(pidx == pf_host[2], axis=1)))}/"
                                                                  f"{pf_host[2].shape[0]}",
                                          "note": "GPU prefill (DECODE routing, residual) against this OpenBLAS run"}
                    pcpu["speedup_gpu"] = round(pcpu["median_ms"] * 1e3 / prefill["us"], 1)
                    prefill["cpu_baseline"] = pcpu
                except Exception as exc:  # report, never hide
                    prefill["cpu_baseline"] = {"error": repr(exc)}
        except Exception as exc:  # report, never hide
            cpu = {"error": repr(exc)}
    elif not args.no_cpu:
        cpu = {"skipped": "the reference CPU leg covers the MoE layers + LM head only (config 5); this run adds "
                          + ", ".join(x for x, on in (("the dense layer", dense), ("sampling rules", sampling),
                                                      ("attention", full)) if on)}
    L.ds_hip_stack_destroy(S)
    if dense:
        L.ds_hip_dense_destroy(dense)
    for A in attns:
        L.ds_hip_attn_destroy(A)
    for h in handles:
        L.ds_hip_layer_destroy(h)

    workload = ((f"whole decoder steps after {args.decoder_step} cached positions: attention "
                 "(10 heads x 128, f32 KV cache) per layer + " if full else "") +
                ("layer-0 dense SwiGLU FFN 1280x6848 bf16 + " if dense else "") +
                (f"repetition penalty {args.repeat_penalty} / no-repeat n-gram {args.no_repeat_ngram} "
                 "after the argmax + " if sampling else "") +
                "config 5: 11 DeepSeek3B-MoE INT8 layers (H1280, 64x[1792x1280 + 1280x896] routed top-6 + 2 shared, "
                f"{'f32 router renormalised' if route == dev.ROUTE_CFG else 'bf16 router, fast-exp softmax over 64'}) "
                f"+ argmax LM head 129280x1280 bf16{' (int8 copy with exact bounds)' if cert else ''}, batch 1; "
                f"{args.steps} timed "
                f"decode steps after {args.warmup} "
                "warm-up steps, each on a fresh seeded input")
    line = {
        "metric": "INT8 MoE decode tok/s (batch 1) + achieved HBM GB/s as % of peak",
        "value": round(args.steps / (ms.value * 1e-3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "ms_per_step_dist": {"median": pct(each, 50), "p10": pct(each, 10), "p90": pct(each, 90), "n": n_each,
                             "method": "graph launches one after another with an event between consecutive "
                                       "launches (launch-to-launch time), after a reset"},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights (u8 codes + f32 scale/offset), f32 accumulate; bf16 LM head" +
                 (" (argmax over an int8 copy with exact bounds, then each block's candidate rows in bf16; the "
                  "same tokens)" if cert else ""),
        "data": "synthetic: seeded N(0,0.02) weights generated on device, seeded N(0,1) f32 hidden states",
        "config": {"workload": workload, "route": args.route, "moe_layer_kernels": layer_kernels,
                   "global_batch": 1, "parallelism": "single GPU"},
        "hbm": {"bytes_per_step": int(bytes_per_step), "achieved_gbs": round(step_gbs, 1),
                "frac_of_peak": round(step_gbs / PEAK_HBM_GBS, 4), "peak_gbs": PEAK_HBM_GBS,
                "frac_of_peak_median": round(bytes_per_step / (pct(each, 50) * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                "wall_s_timed_region": round(wall, 4),
                "bytes_per_step_note": "bytes this implementation reads per step" +
                                       (" (the LM head as its int8 copy)" if cert else ""),
                "one_pass_head_bytes_per_step": int(bytes_per_step - lm_bytes + VOCAB * H * 2),
                "one_pass_head_equivalent_frac_of_peak": round((bytes_per_step - lm_bytes + VOCAB * H * 2) /
                                                               (ms_per_step * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
        "roofline": roofline,
        "roofline_lm_head": roofline_lm,
        "route_cert": route_cert,
        "determinism": {"rerun_tokens_equal": rerun_equal, "of": max(0, hi - lo),
                        "note": "tokens of the timed steps against a second graph run of the same inputs; the "
                                f"{'one-kernel' if layer_kernels == 1 else 'two-kernel'} layers produced both"},
        "kernels": kernel_ms,
        "prefill": prefill,
        "single_configs": singles,
        "decoder_step": decoder,
        "cpu_baseline": cpu,
        "dropin_per_function": dropin,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
