"""Per-kernel measurement of every hot-path function at the GPT-2 124M shapes
(8,192 tokens) on one MI355X -- the MI355X counterpart of the reference's
`flint_bench` (ref bench/harness.cpp:158-288 for the protocol):

  * inputs seeded and resident in HBM; buffer sets rotated so that one pass over
    them exceeds 2x the 256 MB Infinity Cache;
  * HIP-event timing of back-to-back launches after a warm-up, median of
    rounds;
  * absolute TFLOP/s (GEMMs, 2mnk) or GB/s (reductions: each input read once,
    each output written once) and the fraction of MI355X's dense FP16 MFMA
    peak (2,516.6 TFLOP/s) or HBM peak (8 TB/s);
  * beside each figure, the same op in PyTorch: on the GPU (torch.matmul, i.e.
    hipBLASLt, for plain GEMMs -- the reference's "% of cuBLAS" view) and in
    FP32 on the host CPU on a row sample, with the thread count stated.

Used by `bench.py --suite PATH`, or directly:

    python3 -m flint_amd.bench_suite --out suite.json [--only SUBSTRING]

which writes one JSON object per kernel (`--only` keeps the kernels whose name
contains SUBSTRING, or any of a comma-separated list of them, e.g. for a
rocprofv3 counter pass over a few kernels).
"""

import json
import math
import os
import statistics
import time
from pathlib import Path

PEAK_TF = 2516.6
PEAK_GBS = 8000.0
CACHE = 256 << 20
M, C, V, VP, T, H = 8192, 768, 50257, 50304, 1024, 12
B = 8 * H   # attention batch: 8 sequences x 12 heads


def _time_gpu(torch, fn, sets, rounds=5, per_round=None, warmup_s=1.5, sample_ms=100.0):
    """Median per-launch ms over `rounds` samples of back-to-back launches
    (HIP events), after `warmup_s` seconds of launches; each sample holds
    enough launches (a multiple of the buffer sets, at least `per_round`) to
    last `sample_ms` (ref bench/harness.cpp:158-288 for the protocol)."""
    def window(n):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(n):
            fn(sets[i % len(sets)])
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b)

    n = max(per_round or 1, len(sets))
    start = time.perf_counter()
    while True:                       # warm-up, sizing the sample as it goes
        ms = window(n)
        if time.perf_counter() - start >= warmup_s:
            break
        if ms < sample_ms:
            n = min(n * 2, 1 << 20)
    while ms < sample_ms and n < (1 << 20):
        n = max(n + len(sets), int(n * sample_ms / max(ms, 1e-3) * 1.1))
        ms = window(n)
    return statistics.median(window(n) / n for _ in range(rounds))


def _time_cpu(fn, reps=3):
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _nsets(bytes_per_set):
    return max(1, math.ceil(2 * CACHE / max(bytes_per_set, 1)))


def run(f, torch, dev, path, only=None):
    import sys

    sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "tests"))
    from inputs import normal, targets, uniform

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    F = torch.nn.functional
    out = []

    def want(name):
        return not only or any(part in name for part in only.split(","))

    def record(name, kind, work, ms, cpu_s=None, cpu_work=None, peer_ms=None, note=""):
        if kind == "gemm":
            rate = work / (ms * 1e-3) / 1e12
            entry = {"kernel": name, "ms": round(ms, 5), "tflops": round(rate, 1),
                     "frac_mfma_peak": round(rate / PEAK_TF, 4)}
            if cpu_s:
                entry["cpu_fp32_tflops"] = round(cpu_work / cpu_s / 1e12, 4)
            if peer_ms:
                entry["hipblaslt_tflops"] = round(work / (peer_ms * 1e-3) / 1e12, 1)
                entry["vs_hipblaslt"] = round(peer_ms / ms, 3)
        else:
            rate = work / (ms * 1e-3) / 1e9
            entry = {"kernel": name, "ms": round(ms, 5), "gbs": round(rate, 1),
                     "frac_hbm_peak": round(rate / PEAK_GBS, 4)}
            if cpu_s:
                entry["cpu_fp32_gbs"] = round(cpu_work / cpu_s / 1e9, 2)
        entry["cpu_threads"] = threads
        if note:
            entry["note"] = note
        out.append(entry)
        print(json.dumps(entry), flush=True)

    # ---------------------------------------------------------------- GEMMs
    def gemm_case(name, layout, epi, m, n, k, sample_rows=512):
        if not want(name):
            return
        flops = 2 * m * n * k
        per = (m * k + n * k) * 2 + m * n * (4 if epi in ("res", "tn") else 2) * (
            2 if epi in ("gelu", "res") else 1)
        nsets = _nsets(per)
        sets = []
        for r in range(nsets):
            if layout == "tn":
                x = uniform((k, m), 10 * r + 1).to(dev)
                w = uniform((k, n), 10 * r + 2).to(dev)
            elif layout == "nn":
                x = uniform((m, k), 10 * r + 1).to(dev)
                w = normal((k, n), 10 * r + 2, 0.02, torch.float16).to(dev)
            else:
                x = uniform((m, k), 10 * r + 1).to(dev)
                w = normal((n, k), 10 * r + 2, 0.02, torch.float16).to(dev)
            b = normal((n,), 10 * r + 3, 0.02).to(dev)
            ydt = torch.float32 if epi in ("res", "tn") else torch.float16
            y = torch.empty((m, n), dtype=ydt, device=dev)
            aux = None
            if epi == "gelu":
                aux = torch.empty((m, n), dtype=torch.float16, device=dev)
            elif epi == "res":
                aux = normal((m, n), 10 * r + 4).to(dev)
            elif epi == "dgelu":
                aux = normal((m, n), 10 * r + 4, 1.0, torch.float16).to(dev)
            sets.append((x, w, b, y, aux))
        ws = None
        if layout == "tn":
            need = f.gemm_tn_workspace(m, n, k)
            ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev) if need else None

        def call(st):
            x, w, b, y, aux = st
            if layout == "nt":
                if epi == "none":
                    f.gemm_nt(y, x, w, m, n, k)
                elif epi == "bias":
                    f.gemm_nt_bias(y, x, w, b, m, n, k)
                elif epi == "gelu":
                    f.gemm_nt_bias_gelu(y, aux, x, w, b, m, n, k)
                elif epi == "res":
                    f.gemm_nt_bias_residual(y, x, w, b, aux, m, n, k)
            elif layout == "nn":
                if epi == "dgelu":
                    f.gemm_nn_dgelu(y, x, w, aux, m, n, k)
                else:
                    f.gemm_nn(y, x, w, m, n, k)
            else:
                f.gemm_tn(y, x, w, m, n, k, accumulate=True, workspace=ws)

        ms = _time_gpu(torch, call, sets)
        peer = None
        if epi in ("none", "bias", "tn") or layout == "nn" and epi == "none":
            x, w = sets[0][0], sets[0][1]
            if layout == "nt":
                pf = lambda st: torch.matmul(st[0], st[1].T)  # noqa: E731
            elif layout == "nn":
                pf = lambda st: torch.matmul(st[0], st[1])  # noqa: E731
            else:
                pf = lambda st: torch.matmul(st[0].T, st[1])  # noqa: E731
            peer = _time_gpu(torch, pf, sets)
        # CPU fp32 on a row sample of the output.
        rows = min(sample_rows, m)
        xs = sets[0][0].float().cpu()
        ws_ = sets[0][1].float().cpu()
        bs = sets[0][2].cpu()
        if layout == "nt":
            xs = xs[:rows]
            cpu_fn = lambda: F.gelu(xs @ ws_.T + bs, approximate="tanh") if epi == "gelu" else xs @ ws_.T + bs  # noqa: E731,E501
        elif layout == "nn":
            xs = xs[:rows]
            cpu_fn = lambda: xs @ ws_  # noqa: E731
        else:
            xs = xs[:, :rows]
            cpu_fn = lambda: xs.T @ ws_  # noqa: E731
        cpu_s = _time_cpu(cpu_fn, reps=2)
        record(name, "gemm", flops, ms, cpu_s, 2 * rows * n * k, peer,
               note=f"{len(sets)} rotating sets; CPU sample {rows} rows")
        del sets
        torch.cuda.empty_cache()

    gemm_case("flint_gemm_nt_bias qkv 8192x2304x768", "nt", "bias", M, 3 * C, C)
    gemm_case("flint_gemm_nt_bias_gelu mlp-up 8192x3072x768", "nt", "gelu", M, 4 * C, C)
    gemm_case("flint_gemm_nt_bias_residual mlp-down 8192x768x3072", "nt", "res", M, C, 4 * C)
    gemm_case("flint_gemm_nt_bias_residual attn-proj 8192x768x768", "nt", "res", M, C, C)
    gemm_case("flint_gemm_nt logits 8192x50304x768", "nt", "none", M, VP, C, sample_rows=128)
    gemm_case("flint_gemm_nn mlp-up dX 8192x768x3072", "nn", "none", M, C, 4 * C)
    gemm_case("flint_gemm_nn_dgelu 8192x3072x768", "nn", "dgelu", M, 4 * C, C)
    gemm_case("flint_gemm_nn logits dX 8192x768x50304", "nn", "none", M, C, VP, sample_rows=128)
    gemm_case("flint_gemm_tn mlp-up dW 3072x768x8192 (accumulate)", "tn", "tn", 4 * C, C, M)
    gemm_case("flint_gemm_tn attn dW 768x768x8192 (accumulate)", "tn", "tn", C, C, M)
    gemm_case("flint_gemm_tn logits dW 50304x768x8192 (accumulate)", "tn", "tn", VP, C, M,
              sample_rows=128)

    def section_batched():
        # Batched attention GEMMs, 96 heads x 1024 tokens x 64.
        q = uniform((B, T, 64), 1).to(dev)
        kk = uniform((B, T, 64), 2).to(dev)
        s = torch.empty((B, T, T), dtype=torch.float16, device=dev)
        ms = _time_gpu(torch, lambda st: f.gemm_nt_batched(s, q, kk, B, T, T, 64, 0.125), [0])
        record("flint_gemm_nt_batched S=QK^T/8 96x1024x1024x64", "gemm", 2 * B * T * T * 64, ms,
               note="HBM-bound: writes 201 MB")
        p = uniform((B, T, T), 3).to(dev)
        o = torch.empty((B, T, 64), dtype=torch.float16, device=dev)
        ms = _time_gpu(torch, lambda st: f.gemm_nn_batched(o, p, kk, B, T, 64, T), [0])
        record("flint_gemm_nn_batched O=PV 96x1024x64x1024", "gemm", 2 * B * T * T * 64, ms)
        ms = _time_gpu(torch, lambda st: f.gemm_tn_batched(o, p, kk, B, T, 64, T), [0])
        record("flint_gemm_tn_batched dV=P^T dO 96x1024x64x1024", "gemm", 2 * B * T * T * 64, ms)
        del q, kk, s, p, o
        torch.cuda.empty_cache()

    # ----------------------------------------------------------- reductions
    def red_sets(make, per_bytes):
        return [make(r) for r in range(_nsets(per_bytes))]

    def section_layernorm():
        # LayerNorm forward 8192 x 768: x FP32 in, y FP16 + mean/rstd out.
        ln_bytes = M * C * 4 + M * C * 2 + 2 * M * 4 + 2 * C * 4
        sets = red_sets(lambda r: (normal((M, C), r).to(dev), torch.empty((M, C), dtype=torch.float16,
                        device=dev), torch.empty(M, device=dev), torch.empty(M, device=dev)), ln_bytes)
        g = (1 + normal((C,), 9, 0.1)).to(dev)
        bta = normal((C,), 10, 0.1).to(dev)
        ms = _time_gpu(torch, lambda st: f.layernorm_forward(st[1], st[2], st[3], st[0], g, bta, M, C),
                       sets, per_round=64)
        xc = sets[0][0][:2048].cpu()
        cpu_s = _time_cpu(lambda: F.layer_norm(xc, (C,), g.cpu(), bta.cpu()))
        record("flint_layernorm_forward 8192x768", "red", ln_bytes, ms, cpu_s, ln_bytes / 4)
        # LayerNorm backward (accumulate_dx): dy FP16, x FP32, dx FP32 read+write.
        lnb_bytes = M * C * 2 + M * C * 4 + M * C * 4 * 2 + 2 * M * 4 + 3 * C * 4
        wsb = torch.empty(f.layernorm_backward_workspace(M, C), dtype=torch.uint8, device=dev)
        dsets = [(normal((M, C), 20 + r, 1.0, torch.float16).to(dev), torch.zeros((M, C), device=dev))
                 for r in range(len(sets))]
        dg = torch.zeros(C, device=dev)
        db = torch.zeros(C, device=dev)
        ms = _time_gpu(torch, lambda st: f.layernorm_backward(
            st[1][1], dg, db, st[1][0], st[0][0], st[0][2], st[0][3], g, M, C, accumulate_dx=True,
            workspace=wsb), list(zip(sets, dsets)), per_round=64)
        record("flint_layernorm_backward 8192x768 (accumulate_dx)", "red", lnb_bytes, ms,
               note="2 kernels: dbeta + dgamma chunk partials; dx + their merge")
        bg_bytes = M * C * 2 + C * 4
        wsg = torch.empty(f.bias_gradient_workspace(M, 4 * C), dtype=torch.uint8, device=dev)
        dy3 = [normal((M, 4 * C), 30 + r, 1.0, torch.float16).to(dev) for r in range(4)]
        dbias = torch.zeros(4 * C, device=dev)
        ms = _time_gpu(torch, lambda st: f.bias_gradient(dbias, st, M, 4 * C, workspace=wsg), dy3,
                       per_round=64)
        record("flint_bias_gradient 8192x3072", "red", M * 4 * C * 2 + 4 * C * 4, ms)
        del sets, dsets, dy3
        torch.cuda.empty_cache()

    def section_softmax():
        # Causal softmax 96 x 1024 x 1024 (visible half read, full write).
        sm_bytes = B * (T * (T + 1) // 2) * 2 + B * T * T * 2
        ss = [normal((B, T, T), 40 + r, 4.0, torch.float16).to(dev) for r in range(2)]
        pp = [torch.empty((B, T, T), dtype=torch.float16, device=dev) for _ in range(2)]
        ms = _time_gpu(torch, lambda st: f.causal_softmax_forward(pp[st], ss[st], B, T), [0, 1],
                       per_round=16)
        sc = ss[0][:4].float().cpu()
        mask = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
        cpu_s = _time_cpu(lambda: torch.softmax(sc.masked_fill(mask, float("-inf")), -1))
        record("flint_causal_softmax_forward 96x1024x1024", "red", sm_bytes, ms, cpu_s,
               sm_bytes * 4 / B)
        smb_bytes = 2 * B * (T * (T + 1) // 2) * 2 + B * T * T * 2
        ms = _time_gpu(torch, lambda st: f.causal_softmax_backward(ss[st], pp[st], ss[st], B, T,
                                                                   0.125), [0, 1], per_round=16)
        record("flint_causal_softmax_backward 96x1024x1024 (in place)", "red", smb_bytes, ms)
        del ss, pp
        torch.cuda.empty_cache()

    def section_ce():
        # Softmax + cross-entropy 8192 x 50304 (vocab 50257).
        ce_bytes = M * VP * 2 * 2 + M * 2 + M * 4
        lg = normal((M, VP), 50, 2.0, torch.float16).to(dev)
        _, t16 = targets(M, V, 51)
        t16 = t16.to(dev)
        dl = torch.empty_like(lg)
        loss = torch.empty(M, device=dev)
        ms = _time_gpu(torch, lambda st: f.softmax_cross_entropy(dl, loss, lg, t16, 0.125, M, V, VP),
                       [0], per_round=8)
        lc = lg[:256, :V].float().cpu()
        tc = (t16[:256].long() & 0xFFFF).cpu()   # uint16 targets held in int16

        def ce_cpu():
            l_ = lc.clone().requires_grad_(True)
            F.cross_entropy(l_, tc, reduction="sum").backward()

        cpu_s = _time_cpu(ce_cpu)
        record("flint_softmax_cross_entropy 8192x50304", "red", ce_bytes, ms, cpu_s,
               ce_bytes * 256 / M, note="one set (824 MB logits) exceeds the cache")
        del lg, dl
        torch.cuda.empty_cache()

    def section_support():
        # flint_copy over 824 MB: the practical read+write HBM rate of this part,
        # the ceiling the other bandwidth-bound kernels are read against.
        if want("flint_copy"):
            # Copies of the traffic of the reductions above (LN forward, LN
            # backward, softmax, cross-entropy): what a kernel moving that many
            # bytes can reach on this part, launch and ramp included.
            for traffic, label in ((37_748_736, "= LN forward"), (88_080_384, "= LN backward"),
                                   (302_000_000, "= causal softmax forward"),
                                   (2 * M * VP * 2, "= softmax + cross-entropy")):
                nb = traffic // 2 // 16 * 16
                n_ = max(2, -(-(600 << 20) // (2 * nb)))
                src = [torch.ones(nb, dtype=torch.uint8, device=dev) for _ in range(n_)]
                dst = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(n_)]
                ms = _time_gpu(torch, lambda st: f.copy(dst[st], src[st], nb), list(range(n_)),
                               per_round=max(8, n_))
                record(f"flint_copy {2 * nb / 1e6:.0f} MB moved {label}", "red", 2 * nb, ms,
                       note="read + write; the practical HBM ceiling at this size")
                del src, dst
        if want("flint_fp32_to_fp16"):
            count = 124_475_904   # GPT-2 124M parameters, as synced each step
            xs = [normal((count,), 60 + r).to(dev) for r in range(2)]
            ys = torch.empty(count, dtype=torch.float16, device=dev)
            ms = _time_gpu(torch, lambda st: f.fp32_to_fp16(ys, xs[st], count), [0, 1],
                           per_round=8)
            record("flint_fp32_to_fp16 124.5M", "red", count * 6, ms)
            del xs, ys
        if want("flint_heads_split") or want("flint_heads_merge"):
            qkv = [uniform((M, 3 * C), 70 + r).to(dev) for r in range(4)]
            hd = torch.empty((B, T, 64), dtype=torch.float16, device=dev)
            ms = _time_gpu(torch, lambda st: f.heads_split(hd, st, 8, T, H, 64, 3 * C, C), qkv,
                           per_round=16)
            record("flint_heads_split k 8192x2304 -> 96x1024x64", "red", 2 * M * C * 2, ms)
            ms = _time_gpu(torch, lambda st: f.heads_merge(st, hd, 8, T, H, 64, 3 * C, C), qkv,
                           per_round=16)
            record("flint_heads_merge 96x1024x64 -> 8192x2304", "red", 2 * M * C * 2, ms)
            del qkv, hd
        if want("flint_embedding"):
            wte = normal((V, C), 80, 0.02).to(dev)
            wpe = normal((T, C), 81, 0.01).to(dev)
            tok32, tok16 = targets(M, V, 82)
            tok16 = tok16.to(dev)
            xs = [torch.empty((M, C), device=dev) for _ in range(4)]
            emb_bytes = M * C * 4 * 2 + T * C * 4 + M * 2
            ms = _time_gpu(torch, lambda st: f.embedding_forward(st, tok16, wte, wpe, 8, T, V, C),
                           xs, per_round=16)
            record("flint_embedding_forward 8192x768", "red", emb_bytes, ms)
            distinct = int(torch.unique(tok32).numel())
            dx = [normal((M, C), 83 + r).to(dev) for r in range(4)]
            dwte = torch.zeros((V, C), device=dev)
            dwpe = torch.zeros((T, C), device=dev)
            ws = torch.empty(max(f.embedding_backward_workspace(8, T, V, C), 16),
                             dtype=torch.uint8, device=dev)
            ms = _time_gpu(torch, lambda st: f.embedding_backward(
                dwte, dwpe, st, tok16, 8, T, V, C, accumulate_wte=True, accumulate_wpe=True,
                workspace=ws), dx, per_round=16)
            bwd_bytes = M * C * 4 + 2 * distinct * C * 4 + 2 * T * C * 4 + M * 2
            record("flint_embedding_backward 8192x768 (accumulate)", "red", bwd_bytes, ms,
                   note=f"{distinct} distinct tokens; rows read + written once")
            del wte, wpe, xs, dx, dwte, dwpe, ws
        torch.cuda.empty_cache()

    def section_attention():
        # The fused causal attention at GPT-2 124M's shape: 96 batches (8
        # sequences x 12 heads) of 1024 x 64. Work counted as the causal half
        # of the products: forward 2 (S, PV), backward 5 (S recomputed
        # once for P, dP, dV, dK, dQ), 2 * 96 * 64 * 1024^2 / 2 FLOP each.
        Bn, Tn, D = B, T, 64
        half = 2 * Bn * D * Tn * Tn / 2
        sets = []
        for i in range(2):
            q, k, v, g = (normal((Bn, Tn, D), 90 + 4 * i + j, 1.0, torch.float16).to(dev) for j in range(4))
            o = torch.empty_like(q)
            lse = torch.empty((Bn, Tn), device=dev)
            sets.append((q, k, v, g, o, lse, torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)))
        ws = torch.empty(f.attention_backward_workspace(Bn, Tn, D), dtype=torch.uint8, device=dev)
        if want("flint_attention_forward"):
            ms = _time_gpu(torch, lambda st: f.attention_forward(st[4], st[5], st[0], st[1], st[2], Bn, Tn,
                                                                 D, 0.125), sets, per_round=8)
            record("flint_attention_forward causal 96x1024x64", "gemm", 2 * half, ms,
                   note="causal half of S = QK^T and O = PV; scores never stored")
        if want("flint_attention_backward"):
            for st in sets:
                f.attention_forward(st[4], st[5], st[0], st[1], st[2], Bn, Tn, D, 0.125)
            ms = _time_gpu(torch, lambda st: f.attention_backward(st[6], st[7], st[8], st[3], st[0], st[1],
                                                                  st[2], st[4], st[5], Bn, Tn, D, 0.125,
                                                                  workspace=ws), sets, per_round=8)
            record("flint_attention_backward causal 96x1024x64", "gemm", 5 * half, ms,
                   note="causal half of S (recomputed), dP, dV, dK, dQ; deterministic (no atomics)")
        del sets, ws
        torch.cuda.empty_cache()

    def section_gpt2():
        # A whole GPT-2 124M training step: 12 layers, width 768,
        # 12 heads, 8 x 1024 tokens, padded vocabulary 50,304; forward through
        # the loss and backward to every weight gradient, FP16 with loss scale
        # 1024 (dlogits scale 1024 / 8192). 7.00 TFLOP by 2mnk over every GEMM.
        from flint_amd.flint_lib import Gpt2

        L_, S_, T_ = 12, 8, 1024
        for flash in (False, True):
            if want("gpt2_124m_train_step " + ("fused" if flash else "stored")):
                train_step(Gpt2, L_, S_, T_, flash)

    def train_step(Gpt2, L_, S_, T_, flash):
        # flint_gpt2_create's model (the reference's sequence: stored scores
        # and probabilities), then flint_gpt2_create_fused's.
        model = Gpt2(f, L_, H, C, T_, V, VP, S_, T_, backward=True, fused=flash)
        g = torch.Generator().manual_seed(5)
        for name, addr, rows, cols in model.parameters():
            if name.endswith(("ln_1.weight", "ln_2.weight")) or name == "ln_f.weight":
                t = torch.ones(rows, cols)
            elif rows == 1:
                t = torch.zeros(rows, cols)
            else:
                t = torch.randn(rows, cols, generator=g) * 0.02
                if name == "wte.weight":
                    t[V:] = 0
            model.write(addr, t.to(dev))
        model.sync_weights()
        tok = torch.randint(0, V, (S_ * T_,), generator=g).to(torch.int32).to(torch.int16).to(dev)
        tgt = torch.randint(0, V, (S_ * T_,), generator=g).to(torch.int32).to(torch.int16).to(dev)
        scale = 1024.0 / (S_ * T_)

        def step(_):
            model.forward(tok, tgt, scale)
            model.backward(tok)

        ms = _time_gpu(torch, step, [0], rounds=5, per_round=5)
        flops = 7.0013e12
        label = "fused attention" if flash else "stored scores and probabilities"
        entry = {"kernel": f"gpt2_124m_train_step 8x1024 (forward + backward, {label})",
                 "ms": round(ms, 4),
                 "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                 "frac_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_TF, 4),
                 "tokens_per_s": round(S_ * T_ / (ms * 1e-3)), "cpu_threads": threads,
                 "loss": round(model.mean_loss(), 4),
                 "note": "7.00 TFLOP per step (2mnk over every GEMM, attention counted full); "
                         "random-init weights, random tokens"}
        out.append(entry)
        print(json.dumps(entry), flush=True)
        model.close()
        torch.cuda.empty_cache()

    def section_adamw():
        # One clipped, loss-scaled AdamW step over GPT-2 124M's 148 tensors
        # (named_parameters shapes, decay on the matrices): 34 bytes of HBM
        # traffic per parameter (gradient read twice, param/m/v read and
        # written, the FP16 copy written). One set is 4.2 GB, past the cache.
        shapes = [(50257, C), (1024, C)]
        for _ in range(12):
            shapes += [(C,), (C,), (3 * C, C), (3 * C,), (C, C), (C,), (C,), (C,), (4 * C, C), (4 * C,),
                       (C, 4 * C), (C,)]
        shapes += [(C,), (C,)]
        gen = torch.Generator(device=dev).manual_seed(80)
        ts = []
        for shp in shapes:
            n = math.prod(shp)
            ts.append({"param": torch.randn(n, device=dev, generator=gen) * 0.02,
                       "grad": torch.randn(n, device=dev, generator=gen) * 0.1,
                       "exp_avg": torch.zeros(n, device=dev), "exp_avg_sq": torch.zeros(n, device=dev),
                       "param_half": torch.empty(n, dtype=torch.float16, device=dev),
                       "weight_decay": 0.1 if len(shp) == 2 else 0.0})
        total = sum(t["param"].numel() for t in ts)
        state = torch.zeros(8, dtype=torch.float32, device=dev)
        f.train_state_init(state, 1024.0)
        opts = f.adamw_defaults()
        ws = torch.empty(f.adamw_workspace(ts), dtype=torch.uint8, device=dev)
        ms = _time_gpu(torch, lambda _: f.adamw_step(ts, state, opts, ws), [0], per_round=8)
        # CPU: torch's AdamW (foreach) with unscale and clipping on a 4M sample.
        ns = 4 << 20
        cp = [torch.nn.Parameter(torch.randn(ns) * 0.02)]
        cp[0].grad = torch.randn(ns) * 0.1
        copt = torch.optim.AdamW(cp, lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)

        def cpu_step():
            cp[0].grad.mul_(1 / 1024)
            torch.nn.utils.clip_grad_norm_(cp, 1.0)
            copt.step()

        cpu_s = _time_cpu(cpu_step)
        record(f"flint_adamw_step GPT-2 124M ({len(ts)} tensors, {total / 1e6:.1f}M params)", "red",
               34 * total, ms, cpu_s=cpu_s, cpu_work=34 * ns,
               note="3 kernels: gradient norm partials, decision, update + FP16 copy; 34 B/param")
        del ts, ws
        torch.cuda.empty_cache()

    if any(want(x) for x in ("flint_gemm_nt_batched", "flint_gemm_nn_batched",
                             "flint_gemm_tn_batched")):
        section_batched()
    if any(want(x) for x in ("flint_layernorm_forward", "flint_layernorm_backward",
                             "flint_bias_gradient")):
        section_layernorm()
    if any(want(x) for x in ("flint_causal_softmax_forward", "flint_causal_softmax_backward")):
        section_softmax()
    if want("flint_softmax_cross_entropy"):
        section_ce()
    if want("flint_attention_forward") or want("flint_attention_backward"):
        section_attention()
    if want("gpt2_124m_train_step stored") or want("gpt2_124m_train_step fused"):
        section_gpt2()
    if any(want(x) for x in ("flint_copy", "flint_fp32_to_fp16", "flint_heads_split",
                             "flint_heads_merge", "flint_embedding")):
        section_support()
    if want("flint_adamw_step"):
        section_adamw()
    Path(path).write_text(json.dumps(out, indent=1))
    return out


def main():
    import argparse
    import sys

    import torch

    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from flint_amd.flint_lib import Flint

    ap = argparse.ArgumentParser(description="Per-kernel measurement at the GPT-2 124M shapes.")
    ap.add_argument("--out", default="suite.json")
    ap.add_argument("--only", default=None,
                    help="keep kernels whose name contains this (or any of a comma-separated list)")
    a = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("bench_suite needs a GPU")
    run(Flint(), torch, torch.device("cuda:0"), a.out, a.only)


if __name__ == "__main__":
    main()
