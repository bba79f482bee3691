"""Verify-step benchmark of the MI355X target-verify path (one GPU).

Workload (the headline one): a Llama-3-8B-shaped Q4_K_M target (32 layers,
hidden 4096, 32 query / 8 KV heads, head_dim 128, FFN 14336, vocab 128256,
RoPE theta 500000; Q6_K on attn_v / ffn_down in the 16 use_more_bits layers,
Q4_K elsewhere including lm_head), random-init weights N(0, 0.02) synthesised
on the GPU, 512 fp16 KV positions filled with N(0, 1)-like values.

  step = one linear verify of k=4 draft tokens (M=5 rows: the last committed
         token + 4 drafts) with greedy acceptance on the device
         (sd_verify_greedy_linear), then rollback_to() the pre-verify length
         so every step verifies at the same KV length.

The same run also times the 60-node tree verify of the same weights: a
(4,3,2,2,1,1) Cartesian draft tree pruned to 60 nodes (depth 6) over 4096 KV
positions, greedy longest-path acceptance and compaction of the accepted
path's KV rows (sd_verify_greedy_tree + sd_commit_tree_path), then rollback;
the M=1 decode step (observe of one token); an EAGLE-3-style verify (64-node
depth-7 tree over 8192 positions, draft rows in a 32000-token vocabulary
mapped through a seeded injective d2t, rejection sampling at T=1, compaction);
and a Qwen2.5-7B-shaped Q5_K / Q8_0 target with QKV bias verifying k=8 drafts
(M=9) over 2048 positions with rejection sampling at T=1.

Timing: W untimed warmup steps, then K steps bracketed by device
synchronisation.  A second pass of K steps with HIP-event timing on the
decoder's stream gives each dequant-matmul launch's duration, from which the
roofline figure is computed (algorithmic bytes = weight blocks + activations
in + out, per launch).

The CPU baseline times the C restatement of the CPU algorithm candle runs for
a quantised matmul (oracle/cpu_q8k.c: every activation row quantised to Q8_K,
integer Q4_K x Q8_K / Q6_K x Q8_K block dot products scaled in f32, AVX2,
OpenMP over output rows), composed into whole layers, on a bounded sample of
the same step -- one Q6_K-mix layer, one Q4_K layer and the lm_head at M=5,
repeated for about 12 s -- and scales the mean to a whole verify step (16
layers of each kind + lm_head).

roofline.traffic is read from profiles/k1_hbm_traffic_llama8b_q4km.json: the
HBM bytes per launch that rocprofv3's FETCH_SIZE and WRITE_SIZE counters gave
for this workload, scaled by the same counters on a copy kernel.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "abyo-speculate_amd"))

METRIC = "Llama-3-8B Q4_K_M verify-step µs + HBM GB/s at M=5 and 60-node tree"
PEAK_HBM_GBPS = 8000.0
SEED = 0x5EED0002
KV_SEED = 0x4B560002

LLAMA8B = dict(n_layers=32, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
               rope_theta=500000.0, rms_eps=1e-5)
QWEN7B = dict(n_layers=28, hidden=3584, n_heads=28, n_kv_heads=4, head_dim=128, ffn=18944, vocab=152064,
              rope_theta=1000000.0, rms_eps=1e-6)
EAGLE3_PREFIX, EAGLE3_DRAFT_VOCAB = 8192, 32000
QWEN_PREFIX, QWEN_K = 2048, 8


def log(msg: str):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-tree", action="store_true", help="skip the 60-node tree leg")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-ar", action="store_true", help="skip the M=1 decode-step leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the rejection-sampling legs (EAGLE-3 64-node tree at 8192, Qwen2.5-7B M=9 at 2048)")
    ap.add_argument("--prefix", type=int, default=512, help="KV positions before the M=5 verify")
    ap.add_argument("--tree-prefix", type=int, default=4096, help="KV positions before the tree verify")
    return ap.parse_args()


def make_tree(S, root: int, rng: np.random.Generator):
    branching = (4, 3, 2, 2, 1, 1)
    cands = [[int(v) for v in rng.integers(0, LLAMA8B["vocab"], b)] for b in branching]
    lps = [list(np.sort(np.log(rng.dirichlet(np.ones(b))))[::-1].astype(np.float32)) for b in branching]
    full = S.tree_cartesian(root, cands)
    return S.tree_prune(full, lps, 60)


def gemm_rows(prof, classes):
    return [e for e in prof if e[0] in classes]


def draft_rows(rng, n, V, scale=2.0):
    """Draft distributions: softmax of N(0, scale^2) logits (seeded)."""
    z = rng.standard_normal((n, V)) * scale
    z = np.exp(z - z.max(axis=1, keepdims=True))
    return (z / z.sum(axis=1, keepdims=True)).astype(np.float32)


def timed_leg(dec, step, args):
    """(seconds per step, per-launch profile of a second pass, mean of step()'s return)."""
    for _ in range(args.warmup):
        step()
    dec.synchronize()
    t0 = time.perf_counter()
    acc = 0.0
    for _ in range(args.steps):
        acc += step()
    dec.synchronize()
    t = (time.perf_counter() - t0) / args.steps
    dec.profile_enable(True)
    for _ in range(args.steps):
        step()
    dec.synchronize()
    prof = dec.profile_read()
    dec.profile_enable(False)
    return t, prof, acc / args.steps


def wall_per_step(dec, step, args):
    """Seconds per step of step() (warm-up, then the leg's step count), no profile."""
    for _ in range(args.warmup):
        step()
    dec.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dec.synchronize()
    return (time.perf_counter() - t0) / args.steps


def leg_summary(t, prof, tokens_per_step, extra):
    g = gemm_rows(prof, ("qkv", "wo", "gate_up", "down", "lm_head"))
    b = sum(e[1] for e in g)
    tt = sum(e[2] for e in g) * 1e-3
    out = {"us": round(t * 1e6, 1), "tokens_per_s": round(tokens_per_step / t, 1),
           "k1_gbps": round(b / tt / 1e9, 1), "k1_frac": round(b / tt / 1e9 / PEAK_HBM_GBPS, 4),
           "k1_avg_launch_us": round(tt / len(g) * 1e6, 2), "kernels": summarize(prof)}
    out.update(extra)
    return out


def summarize(prof):
    out = {}
    for cls in ("qkv", "wo", "gate_up", "down", "lm_head", "attn", "qkv_attn"):
        es = [e for e in prof if e[0] == cls]
        if not es:
            continue
        b = sum(e[1] for e in es)
        t = sum(e[2] for e in es) * 1e-3
        out[cls] = {"launches": len(es), "avg_us": round(t / len(es) * 1e6, 2),
                    "gbps": round(b / t / 1e9, 1)}
    return out


CPU_SAMPLE_S = 12.0
TRAFFIC_FILE =os.path.join(ROOT, "profiles", "k1_hbm_traffic_llama8b_q4km.json")


def measured_traffic(leg: str):
    """HBM bytes per dequant-matmul launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes over this workload (copy-kernel calibrated), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return int(t[leg]["traffic_bytes_per_launch"]), os.path.relpath(TRAFFIC_FILE, ROOT)
    except (OSError, KeyError, ValueError):
        return None, None


def cpu_baseline():
    """The CPU restatement of candle's quantised matmul path (Q8_K activations,
    integer block dot products, AVX2, OpenMP over rows) in whole layers -- norms,
    Q/K/V, RoPE, attention over 512 cached positions, wo, SwiGLU MLP, residuals --
    timed on a bounded sample and scaled to one M=5 verify step."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    if not os.path.exists(O.LIB_PATH):
        import build_oracle
        build_oracle.build()
    import cpu_baseline as CB
    cfg = O.ModelConfig(arch="llama", mix="q4_k_m", seed=SEED, ctx_len=1024, **LLAMA8B)
    t_start = time.perf_counter()
    r = CB.time_step_sample(cfg, 512, 5, CPU_SAMPLE_S)
    log(f"cpu baseline: {r['reps']} repetitions; Q6_K-mix layer {r['q6_layer_s'] * 1e3:.1f} ms, Q4_K layer "
        f"{r['q4_layer_s'] * 1e3:.1f} ms, lm_head {r['lm_head_s'] * 1e3:.1f} ms")
    return {"value": round(r["step_s"] * 1e6, 1), "unit": "us/verify (M=5)", "cores": CB.threads(), "kind": "port",
            "cpu": CB.cpu_model(),
            "sample": f"CPU restatement of candle's CPU QMatMul path (per-row Q8_K activation quantisation, "
                      f"integer Q4_K/Q6_K x Q8_K block dot products with f32 scaling, AVX2, OpenMP over output "
                      f"rows) in whole layers at M=5 over 512 cached positions (f32 attention, RMSNorm, RoPE, "
                      f"SwiGLU, residuals): one Q6_K-mix layer, one Q4_K layer and the final norm + Q4_K lm_head "
                      f"of the same synthetic weights, {r['reps']} repetitions "
                      f"({time.perf_counter() - t_start:.1f} s), mean scaled to {r['n_q6_layers']}+"
                      f"{cfg.n_layers - r['n_q6_layers']} layers + lm_head"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the verify step of one batch-1 decoder "
              "runs on a single MI355X", file=sys.stderr)
        sys.exit(2)
    import speculate_hip as S
    if not os.path.exists(S.LIB_PATH):
        sys.path.insert(0, ROOT)
        import __graft_entry__
        __graft_entry__.build()
    S.load_library()

    ctx = max(args.prefix + 8, args.tree_prefix + 64,
              0 if args.no_extra else EAGLE3_PREFIX + 72 + 8 * (args.steps + args.warmup)) + 64
    cfg = S.Config(arch=S.ARCH_LLAMA, ctx_len=ctx, max_batch=64, **LLAMA8B)
    log(f"creating decoder (ctx {ctx}) and synthesising Q4_K_M weights")
    dec = S.HipQuantDecoder(cfg)
    dec.synthesize(S.MIX_Q4_K_M, SEED, 0.02)
    rng = np.random.default_rng(SEED)

    # ---------------- M=5 linear verify ----------------
    hist = [int(v) for v in rng.integers(0, cfg.vocab, args.prefix + 1)]
    dec.prime_synthetic(hist, KV_SEED)
    drafts = [int(v) for v in rng.integers(0, cfg.vocab, 4)]
    n0 = len(hist)

    def step_linear():
        commits, acc = dec.verify_greedy_linear(drafts)
        dec.rollback_to(n0)
        return commits, acc

    log(f"M=5 verify: {args.warmup} warmup + {args.steps} timed steps at KV {args.prefix}")
    for _ in range(args.warmup):
        step_linear()
    dec.synchronize()
    t0 = time.perf_counter()
    accepted = 0
    for _ in range(args.steps):
        _, acc = step_linear()
        accepted += acc
    dec.synchronize()
    t_lin = (time.perf_counter() - t0) / args.steps
    log(f"M=5 verify: {t_lin * 1e6:.1f} us/step")

    dec.profile_enable(True)
    for _ in range(args.steps):
        step_linear()
    dec.synchronize()
    prof = dec.profile_read()
    dec.profile_enable(False)
    gem = gemm_rows(prof, ("qkv", "wo", "gate_up", "down", "lm_head"))
    gb = sum(e[1] for e in gem)
    gt = sum(e[2] for e in gem) * 1e-3
    per_launch_bytes = gb / len(gem)
    avg_launch_s = gt / len(gem)
    achieved = per_launch_bytes / avg_launch_s / 1e9
    # every profiled launch: the K1 matmuls, and the attention alone or fused
    # with the Q/K/V matmul (qkv_attn: its weights, activations, outputs and
    # cache rows)
    step_bytes = sum(e[1] for e in prof) / args.steps
    log(f"K1 dequant-matmul: {achieved:.0f} GB/s over {len(gem)} launches")
    traffic, traffic_src = measured_traffic("m5")

    result = {
        "metric": METRIC, "value": round(t_lin * 1e6, 1), "unit": "us", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(t_lin * 1e3, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_k/q6_k weights, fp16 MFMA, f32 accumulate",
        "data": "synthetic (random-init N(0,0.02) weights quantised on the GPU, N(0,1) fp16 KV)",
        "config": {"workload": "Llama-3-8B-shaped Q4_K_M verify step, M=5 (k=4 drafts), KV 512 fp16, greedy "
                               "acceptance on the device",
                   "layers": 32, "hidden": 4096, "heads": "32q/8kv", "ffn": 14336, "vocab": 128256,
                   "M": 5, "kv_positions": args.prefix},
        "verify_steps_per_s": round(1.0 / t_lin, 1),
        "tokens_per_s": round((accepted / args.steps + 1) / t_lin, 1),
        "step_hbm_gbps": round(step_bytes / t_lin / 1e9, 1),
        "step_algorithmic_bytes": int(step_bytes),
        "kernels": summarize(prof),
        "roofline": {"bound": "hbm",
                     "kernel": f"k_qmm (K1 fused dequant-matmul for M<=16: the {len(gem) // args.steps} matmul-only "
                               "launches of a step; the Q/K/V matmul runs inside the fused Q/K/V + attention "
                               "launch, kernels.qkv_attn)",
                     "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "bytes_per_launch": int(per_launch_bytes), "avg_launch_us": round(avg_launch_s * 1e6, 2)},
    }

    # ---------------- M=1 decode step (what autoregressive decoding runs per token) ----------------
    if not args.no_ar:
        dec.rollback_to(n0)

        def step_ar():
            dec.observe(drafts[:1])
            dec.rollback_to(n0)

        for _ in range(args.warmup):
            step_ar()
        dec.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step_ar()
        dec.synchronize()
        t_ar = (time.perf_counter() - t0) / args.steps
        log(f"M=1 decode step: {t_ar * 1e6:.1f} us")
        result["ar_m1"] = {"us": round(t_ar * 1e6, 1), "tokens_per_s": round(1.0 / t_ar, 1),
                           "kv_positions": args.prefix,
                           "what": "observe of one token: M=1 forward with the lm_head row (the step an "
                                   "autoregressive decoder runs per token, logits left on the device)"}

    # ---------------- 60-node tree verify ----------------
    if not args.no_tree:
        hist = [int(v) for v in rng.integers(0, cfg.vocab, args.tree_prefix + 1)]
        dec.prime_synthetic(hist, KV_SEED + 1)
        toks, pars = make_tree(S, hist[-1], rng)
        n1 = len(hist)
        tree = (toks, pars)

        def step_tree():
            path, bonus, bnode = dec.verify_greedy_tree(tree)
            dec.commit_tree_path(tree, path)
            dec.rollback_to(n1)
            return path

        log(f"tree verify: {len(toks)} nodes at KV {args.tree_prefix}")
        for _ in range(args.warmup):
            step_tree()
        dec.synchronize()
        t0 = time.perf_counter()
        plen = 0
        for _ in range(args.steps):
            plen += len(step_tree())
        dec.synchronize()
        t_tree = (time.perf_counter() - t0) / args.steps
        dec.profile_enable(True)
        for _ in range(args.steps):
            step_tree()
        dec.synchronize()
        tprof = dec.profile_read()
        dec.profile_enable(False)
        tg = gemm_rows(tprof, ("qkv", "wo", "gate_up", "down", "lm_head"))
        tb = sum(e[1] for e in tg)
        tt = sum(e[2] for e in tg) * 1e-3
        # the step's algorithmic bytes as for the M=5 leg: every K1 launch's weight blocks, activations
        # and outputs, plus the K/V rows each layer's attention reads once
        tstep_bytes = (tb + sum(e[1] for e in tprof if e[0] == "attn")) / args.steps
        log(f"tree verify: {t_tree * 1e6:.1f} us/step ({tstep_bytes / t_tree / 1e9:.0f} GB/s over the step), "
            f"K1 {tb / tt / 1e9:.0f} GB/s")
        result["tree60"] = {"us": round(t_tree * 1e6, 1), "nodes": int(len(toks)), "kv_positions": args.tree_prefix,
                            "tokens_per_s": round((plen / args.steps) / t_tree, 1),
                            "step_hbm_gbps": round(tstep_bytes / t_tree / 1e9, 1),
                            "step_algorithmic_bytes": int(tstep_bytes),
                            "k1_gbps": round(tb / tt / 1e9, 1),
                            "k1_frac": round(tb / tt / 1e9 / PEAK_HBM_GBPS, 4),
                            "k1_kernel": "k_qgx (K1 for M>16)",
                            "k1_bytes_per_launch": int(tb / len(tg)),
                            "k1_avg_launch_us": round(tt / len(tg) * 1e6, 2),
                            "k1_traffic": measured_traffic("tree60")[0],
                            "kernels": summarize(tprof)}

    if not args.no_extra:
        # ---------------- EAGLE-3 verify: 64-node tree at 8192, d2t, rejection ----------------
        erng = np.random.default_rng(SEED + 5)
        Vd = EAGLE3_DRAFT_VOCAB
        d2t = erng.choice(cfg.vocab, size=Vd, replace=False).astype(np.int64)
        dec.set_d2t(d2t)
        hist = [int(v) for v in erng.integers(0, cfg.vocab, EAGLE3_PREFIX + 1)]
        dec.prime_synthetic(hist, KV_SEED + 2)
        n1 = len(hist)
        cand_d = [[int(v) for v in erng.choice(Vd, b, replace=False)] for b in (4, 3, 2, 2, 1, 1, 1)]
        lps = [list(np.sort(np.log(erng.dirichlet(np.ones(len(c)))))[::-1].astype(np.float32)) for c in cand_d]
        etree = S.tree_prune(S.tree_cartesian(hist[-1], [[int(d2t[v]) for v in c] for c in cand_d]), lps, 64)
        ne = len(etree[0])
        q_d = draft_rows(erng, ne, Vd)
        u = [float(x) for x in erng.random(ne, dtype=np.float32)]

        # the draft rows stay on the device, where a GPU draft model leaves them
        q_dev = S.DeviceArray(q_d)

        def step_e3():
            path, tok, used = dec.verify_rejection_tree_device(etree, q_dev.ptr, ne, Vd, list(range(ne)), u, 1.0)
            dec.commit_tree_path(etree, path)
            dec.rollback_to(n1)
            return len(path)

        def step_e3_host():
            path, tok, used = dec.verify_rejection_tree(etree, q_d, list(range(ne)), u, 1.0)
            dec.commit_tree_path(etree, path)
            dec.rollback_to(n1)
            return len(path)

        log(f"EAGLE-3 verify: {ne}-node tree at KV {EAGLE3_PREFIX}, d2t {Vd} -> {cfg.vocab}, rejection at T=1")
        t_e3, eprof, plen = timed_leg(dec, step_e3, args)
        t_e3h = wall_per_step(dec, step_e3_host, args)
        q_dev.close()
        log(f"EAGLE-3 verify: {t_e3 * 1e6:.1f} us/step (draft rows uploaded per step: {t_e3h * 1e6:.1f})")
        result["eagle3_tree64"] = leg_summary(
            t_e3, eprof, plen,
            {"nodes": ne, "kv_positions": EAGLE3_PREFIX, "draft_vocab": Vd,
             "us_host_draft_rows": round(t_e3h * 1e6, 1),
             "what": "tree forward (K1 M=64, tree attention over 8192 positions), rejection walk over the d2t-mapped "
                     "draft rows (64 x 32000 f32 resident on the device; us_host_draft_rows: uploaded from pageable "
                     "host memory per step), compaction of the accepted path"})

        # ---------------- EAGLE-3 draft round on the device (the producer of that tree) ----------------
        log("EAGLE-3 draft: LLaMA3.1-8B-shaped f16 draft (hidden 4096, FFN 14336, 32000-token head), synthesised")
        # RoPE tables past the 8192 committed positions (the checkpoint's 2048 would end the round there)
        dr = S.HipEagle3Draft(target_vocab=cfg.vocab, max_pos=EAGLE3_PREFIX + 64 + 8 * (args.steps + args.warmup))
        dr.synthesize(SEED + 7, 0.02)
        dr.set_tensor(S.D3_D2T, d2t)
        ks = (4, 3, 2, 2, 1, 1, 1)
        layers = S.default_layers_for(cfg.n_layers)

        def step_draft():
            ids, lp, _ = dr.round(dec, layers, len(ks), list(ks))
            return len(ids)

        # the first round computes the committed token's rows (an M=1 forward over 8192 positions); from then
        # on a one-token observe collects them as it goes, and repeated rounds at one state reuse them
        t_dr = wall_per_step(dec, step_draft, args)

        # the whole run_eagle3 iteration (eagle3.rs:586-790): draft round, Cartesian tree pruned to 64 nodes,
        # tree verify with greedy acceptance, commit of the accepted path, observe of the bonus token
        root = [hist[-1]]
        grown = [0]

        def step_loop():
            ids, lp, _ = dr.round(dec, layers, len(ks), list(ks))
            tree = S.tree_prune(S.tree_cartesian(root[0], ids), lp, 64)
            path, bonus, _ = dec.verify_greedy_tree(tree)
            dec.commit_tree_path(tree, path)
            dec.observe([bonus])
            root[0] = bonus
            grown[0] += len(path)
            return len(path)

        t_loop = wall_per_step(dec, step_loop, args)
        per_it = grown[0] / (args.warmup + args.steps)
        dec.rollback_to(n1)
        wb = sum(dr.tensor_bytes(k) for k in range(S.D3_FC + 1, S.D3_LM_HEAD + 1))
        rb = dr.tensor_bytes(S.D3_FC) + len(ks) * wb
        log(f"EAGLE-3 draft round: {t_dr * 1e6:.1f} us (depth {len(ks)}, top-k {ks}, layers {layers}); "
            f"whole iteration {t_loop * 1e6:.1f} us, {per_it:.2f} tokens each")
        result["eagle3_draft_round"] = {
            "us": round(t_dr * 1e6, 1), "depth": len(ks), "top_k": list(ks), "layers": layers,
            "draft_weight_bytes": int(rb),
            "draft_weight_gbps_incl_collect": round(rb / t_dr / 1e9, 1),
            "iteration_us": round(t_loop * 1e6, 1), "tokens_per_iteration": round(per_it, 3),
            "iteration_tokens_per_s": round(per_it / t_loop, 1),
            "what": "us: one draft round of run_eagle3 on the device -- the committed token's hidden states after 3 "
                    "layers (collected by the one-token observe that appended it), 7 midlayer steps (fc on the "
                    "first), norm + lm_head over 32000 ids, top-k, log-probs and d2t, one host copy of the results; "
                    "iteration_us: the whole loop iteration -- that round, the Cartesian tree pruned to 64 nodes, "
                    "tree verify over ~8200 positions with greedy acceptance, commit of the path, observe of the bonus "
                    "(random weights: the target accepts ~nothing, so about one token per iteration)"}
        dr.close()

        # ---------------- EAGLE-2 draft round on the device (EAGLE-LLaMA3-Instruct-8B shapes) ----------------
        log("EAGLE-2 draft: LLaMA3-8B-shaped f16 draft (own 128256-token table, the target's lm_head), synthesised")
        d2 = S.HipEagleDraft(vocab=cfg.vocab, max_pos=EAGLE3_PREFIX + 256)
        d2.synthesize(SEED + 9, 0.02)
        ks2 = (4, 3, 2, 2, 1, 1)
        th = dec.last_hidden_state()

        def step_draft2():
            ids, lp = d2.round(dec, th, len(ks2), list(ks2))
            return len(ids)

        t_d2 = wall_per_step(dec, step_draft2, args)
        wb2 = sum(d2.tensor_bytes(k) for k in range(S.D2_FC, S.D2_POST_NORM + 1))
        lmb = cfg.vocab * cfg.hidden // 256 * 144  # Q4_K: 144 bytes per 256 weights
        log(f"EAGLE-2 draft round: {t_d2 * 1e6:.1f} us (depth {len(ks2)}, top-k {ks2})")
        result["eagle2_draft_round"] = {
            "us": round(t_d2 * 1e6, 1), "depth": len(ks2), "top_k": list(ks2),
            "draft_weight_bytes_per_step": int(wb2), "target_lm_head_bytes_per_step": lmb,
            "what": "one draft round of run_eagle on the device from the committed token's final-norm hidden state "
                    "(8193 positions): per step the draft's embedding row, fc over [hidden, embedding], one f16 "
                    "Llama block, the target's Q4_K lm_head (128256 x 4096) on the output, top-k over 128256 "
                    "logits with log-probs; the tree60 leg's branching (4,3,2,2,1,1)"}
        d2.close()
    dec.close()

    if not args.no_extra:
        # ---------------- Qwen2.5-7B-shaped Q5_K/Q8_0, M=9 at 2048, rejection ----------------
        qcfg = S.Config(arch=S.ARCH_QWEN2, ctx_len=QWEN_PREFIX + 128, max_batch=64, **QWEN7B)
        log("creating the Qwen2.5-7B-shaped decoder (Q5_K attention, Q8_0 FFN, QKV bias)")
        qd = S.HipQuantDecoder(qcfg)
        qd.synthesize(S.MIX_Q5K_Q80, SEED, 0.02)
        qrng = np.random.default_rng(SEED + 3)
        hist = [int(v) for v in qrng.integers(0, qcfg.vocab, QWEN_PREFIX + 1)]
        qd.prime_synthetic(hist, KV_SEED + 3)
        n0q = len(hist)
        q = draft_rows(qrng, QWEN_K, qcfg.vocab)
        qdrafts = [int(qrng.choice(qcfg.vocab, p=r.astype(np.float64) / r.astype(np.float64).sum())) for r in q]
        uq = [float(x) for x in qrng.random(QWEN_K + 1, dtype=np.float32)]

        q_dev = S.DeviceArray(q)

        def step_q():
            commits, n_acc, used = qd.verify_rejection_linear_device(qdrafts, q_dev.ptr, uq, 1.0)
            qd.rollback_to(n0q)
            return len(commits)

        def step_q_host():
            commits, n_acc, used = qd.verify_rejection_linear(qdrafts, q, uq, 1.0)
            qd.rollback_to(n0q)
            return len(commits)

        def step_q_greedy():
            qd.verify_greedy_linear(qdrafts)
            qd.rollback_to(n0q)
            return 0

        log(f"Qwen2.5-7B verify: M={QWEN_K + 1} at KV {QWEN_PREFIX}, rejection at T=1")
        t_q, qprof, ncom = timed_leg(qd, step_q, args)
        t_qh = wall_per_step(qd, step_q_host, args)
        t_qg = wall_per_step(qd, step_q_greedy, args)
        q_dev.close()
        log(f"Qwen2.5-7B verify: {t_q * 1e6:.1f} us/step (draft rows uploaded per step: {t_qh * 1e6:.1f}; "
            f"greedy acceptance: {t_qg * 1e6:.1f})")
        result["qwen7b_m9"] = leg_summary(
            t_q, qprof, ncom,
            {"M": QWEN_K + 1, "kv_positions": QWEN_PREFIX,
             "us_host_draft_rows": round(t_qh * 1e6, 1), "us_greedy_acceptance": round(t_qg * 1e6, 1),
             "rejection_overhead_us": round((t_q - t_qg) * 1e6, 1),
             "what": "linear verify of 8 drafts (K1 M=9 on Q5_K / Q8_0 with QKV bias), rejection walk over "
                     "8 x 152064 f32 draft rows resident on the device (us_host_draft_rows: uploaded from pageable "
                     "host memory per step; rejection_overhead_us: over the same verify with greedy acceptance)"})
        qd.close()

    if not args.no_cpu:
        log("CPU baseline (bounded sample)")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
