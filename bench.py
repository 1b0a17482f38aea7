#!/usr/bin/env python3
"""Benchmark of the decode-time sampler on one MI355X.

A step is one sampler call over one batch of seeded synthetic input.  The
default workload is the headline configuration C2 (B=64, V=128256 fp32:
penalties from a 512-id history, temperature, top-k 50, top-p 0.9, one host
uniform per row); `--workload` selects one of the other configurations of the
same generator set (tinygpt_amd/workloads.py):

  c1  B=1, V=256 byte-level sampling (latency-bound)
  c2  B=64, V=128256 fp32, full chain (headline)
  c2m C2 plus the grammar mask stage (1024-state table of C3's statistics):
      the north star's full penalty + mask + top-k/top-p + draw chain
  c3  B=128, V=32000 fp32, grammar mask table of 4096 states, greedy + top-p
  c4  B=1024, V=151936 bf16, per-row top-k/top-p/T/repetition
  c5  B=32 sequences, k=8 draft tokens, V=128256 speculative verification
  lp  teacher-forced token log-probabilities: 2048 positions, V=128256 fp32
      (tgs_token_logprobs; a row outside the sampling chain)
  mask  grammar mask rows built on the device (tgs_mask_rows_from_dfa): 64
      new tool-tag FSM states per call over a 151,936-token byte vocabulary
  jsondec  JSON-schema constrained decoding, 64 sequences under the v11 schema:
      per step the batch's mask rows (new ones built on the device), one
      sampling call over the masked logits, and the commit of the sampled
      tokens; timed eagerly (host work inside each step)
  json  JSON-schema grammar rows: 64 new snapshots of the reference's
      pace-fm-response-v11 schema per call, local DFA on the host and rows on
      the device (tinygpt_amd.json_schema), V=151,936; timed eagerly (host work
      inside each call)
  read  the plain read of C2's logits with the fused kernel's grid and load
      pattern (libtgs_floor.so): the floor under the headline.  The default
      c2 line carries it and c2m as sub-objects ("read_floor", "c2m"), timed
      the same way (--no-c2m leaves both out)

Inputs are resident in HBM before timing; distinct input sets rotate so the
256 MB Infinity Cache cannot serve repeats (at least 512 MB in rotation
where a set is large).  The calls are captured in one HIP graph of --steps calls
cycling over the sets (above 4096 steps: a graph of at most 4096 calls
replayed, plus one graph of the remainder) so that exactly --steps calls are
timed; an untimed replay of the same graph goes first, so the timed calls
queue behind GPU work as they would behind a model's forward pass.  The timed
region is bracketed by synchronisations and HIP events on the launch stream.  Then 256 eager calls, each between two HIP events, give the per-call
p10 / p50 / p90.

Prints one JSON line with the roofline of the call, the CPU oracle timed on
this host over a bounded sample, and the parity report of the sampled
outputs against the oracle on the same inputs: id agreement, kept-set and
top-p count agreement, the largest relative error of the reported
probabilities against fp64 softmax of the canonical logits, and the draw /
top-p boundary cases (u or p within 1e-6 of a CDF step) with the
disagreements outside them.

`--calibrate-copy MIB` instead runs a plain device-to-device copy of MIB MiB
a few times: profiling it with the FETCH_SIZE / WRITE_SIZE counters gives the
scale between those counters and bytes actually moved, which converts the
sampling kernel's counter readings into HBM bytes per launch.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "sampled rows/sec @B=64,V=128256 full chain; HBM GB/s as % of peak"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="c2",
                    choices=["c1", "c2", "c2m", "c3", "c4", "c5", "lp", "mask", "json", "jsondec", "read"])
    ap.add_argument("--no-c2m", action="store_true", help="leave the masked chain out of the default c2 line")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of graph replay")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run only a plain copy of MIB MiB (counter calibration)")
    return ap.parse_args()


def oracle_mod():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle

    pyoracle.build()
    return pyoracle


def cpu_threads():
    """Threads of the CPU baseline: every core this process may run on, at
    most 16 (a one-GPU box's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def timed_loop(fn, n_sets, seconds):
    """Calls fn(i) over the sets for about `seconds`; returns (units/s, units, outputs by set)."""
    units = 0
    outs = {}
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds or units == 0:
        o, n = fn(i % n_sets)
        outs[i % n_sets] = o
        units += n
        i += 1
    return units / (time.perf_counter() - t0), units, outs


# ---------------------------------------------------------------- workloads
class Sampling:
    """c1-c4: one tgs_sample call per step over one batch."""

    def __init__(self, name, torch, tg, W):
        self.name = name
        self.torch = torch
        dev = "cuda:0"
        if name == "c1":
            self.rot, self.B, self.V, self.H = 16, 1, 256, 64
            c1 = W.config1_step_inputs(steps=self.rot, V=self.V, H=self.H)
            self.sets = [dict(logits=c1["logits"][i:i + 1].copy(), params=c1["params"], u=c1["u"][i:i + 1].copy(),
                              hist=c1["hist0"][None, :].copy(), hist_len=np.array([self.H], np.int32),
                              mask_table=None) for i in range(self.rot)]
            self.config = {"workload": "c1_byte_level", "B": 1, "V": 256, "history": 64, "top_k": 40, "top_p": 0.95,
                           "temperature": 0.8, "repetition": 1.1}
            self.dtype = "f32"
        elif name == "c2":
            self.rot, self.B, self.V, self.H = 16, 64, 128256, 512
            self.sets = [W.config2(B=self.B, V=self.V, H=self.H, seed_offset=i * 1000) for i in range(self.rot)]
            self.config = {"workload": "c2_llama3_bpe", "B": 64, "V": 128256, "history": 512, "top_k": 50,
                           "top_p": 0.9, "temperature": 0.7, "presence": 0.5, "frequency": 0.3}
            self.dtype = "f32"
        elif name == "c2m":
            self.rot, self.B, self.V, self.H = 16, 64, 128256, 512
            g = W.rng(20)
            table = W.mask_table_loguniform(g, 1024, self.V)
            self.sets = []
            for i in range(self.rot):
                s = W.config2(B=self.B, V=self.V, H=self.H, seed_offset=i * 1000)
                s["mask_table"] = table
                s["params"]["mask_state"] = g.integers(0, table.shape[0], size=self.B).astype(np.int32)
                self.sets.append(s)
            self.config = {"workload": "c2m_full_chain_masked", "B": 64, "V": 128256, "history": 512, "top_k": 50,
                           "top_p": 0.9, "temperature": 0.7, "presence": 0.5, "frequency": 0.3,
                           "mask_states": 1024, "mask_density": "log-uniform [0.1%, 30%]"}
            self.dtype = "f32"
        elif name == "c3":
            self.rot, self.B, self.V, self.H = 16, 128, 32000, 0
            base = W.config3(B=self.B, V=self.V)
            self.sets = [base]
            g = np.random.default_rng(W.SEED_BASE + 3 + 7777)
            for i in range(1, self.rot):
                s = dict(base)
                s["logits"] = W.normal_f32(g, (self.B, self.V), 2.5)
                p = base["params"].copy()
                p["mask_state"] = g.integers(0, base["mask_table"].shape[0], size=self.B).astype(np.int32)
                s["params"] = p
                s["u"] = W.uniforms(g, self.B)
                self.sets.append(s)
            self.config = {"workload": "c3_grammar", "B": 128, "V": 32000, "mask_states": 4096,
                           "greedy_rows": 64, "top_p": 0.95, "temperature": 1.0}
            self.dtype = "f32"
        else:  # c4
            self.rot, self.B, self.V, self.H = 2, 1024, 151936, 256
            self.sets = [W.config4(B=self.B, V=self.V, H=self.H, seed_offset=i * 1000) for i in range(self.rot)]
            self.config = {"workload": "c4_large_batch_bf16", "B": 1024, "V": 151936, "history": 256,
                           "top_k": "U{1..1024}", "top_p": "U[0.5,1]", "temperature": "U[0.3,1.5]",
                           "repetition": "U[1.05,1.3]"}
            self.dtype = "bf16 (upcast to f32)"
        mt = self.sets[0].get("mask_table")
        self.sampler = tg.Sampler(device=0, max_batch=self.B, max_vocab=self.V, max_hist=max(self.H, 1))
        if mt is not None:
            self.sampler.set_mask_table(mt, self.V)
        else:
            self.sampler.set_mask_table(np.zeros((0, 1), np.uint32), 1)
        self.d = []
        for s in self.sets:
            lg = s["logits"]
            t = torch.from_numpy(lg).to(dev)
            if lg.dtype == np.uint16:
                t = t.view(torch.bfloat16)
            self.d.append(dict(
                logits=t,
                params=tg.params_to_device(s["params"], dev),
                u=torch.from_numpy(s["u"]).to(dev),
                hist=None if s.get("hist") is None else torch.from_numpy(s["hist"]).to(dev),
                hist_len=None if s.get("hist_len") is None else torch.from_numpy(s["hist_len"]).to(dev),
                out=torch.empty(self.B, dtype=torch.int32, device=dev),
            ))
        self.hints = [tg.batch_hint(s["params"], self.V) for s in self.sets]
        self.alg_bytes = W.algorithmic_bytes_per_row(name, self.V, self.H, dtype_bytes=2 if name == "c4" else 4) * self.B
        self.units_per_step = self.B
        self.unit = "rows/s"
        self.metric = METRIC if name == "c2" else f"sampled rows/sec, workload {self.config['workload']}"

    def launch(self, i, stream):
        x = self.d[i % self.rot]
        self.sampler.sample(x["logits"], x["params"], x["u"], hist=x["hist"], hist_len=x["hist_len"],
                            out=x["out"], stream=stream, hint=self.hints[i % self.rot])

    def gpu_outputs(self):
        return {i: self.d[i]["out"].cpu().numpy() for i in range(self.rot)}

    def parity_report(self, pyoracle, nthreads, n_sets=4, max_rows=128):
        """The first n_sets sets (at most max_rows rows each), sampled once more
        with the diagnostic outputs, against the oracle on the same rows:
        ids; the top-k / top-p sizes, masses and cut ids; the kept sets and
        reported probabilities of rows that report a kept list (greedy rows
        and rows with 1 <= top_k <= 1024); the largest relative error of
        those probabilities against fp64 softmax of the oracle's canonical
        logits over the top-p survivors; the boundary cases."""
        import torch

        import tinygpt_amd as tg

        dev = "cuda:0"
        kc = 64 if self.name in ("c1", "c2", "c2m") else 1024
        R = min(self.B, max_rows)
        rep = dict(rows=0, ids_equal=0, topk_topp_equal=0, kept_rows=0, kept_equal=0, prob_rows=0,
                   probs_bit_equal_oracle=0, max_rel_prob_err_fp64=0.0, draw_boundary=0, topp_boundary=0,
                   id_disagreements_outside_boundary=0)
        for i in range(min(n_sets, self.rot)):
            x, s = self.d[i], self.sets[i]
            dbg = dict(kept_ids=torch.full((self.B, kc), -7, dtype=torch.int32, device=dev),
                       kept_probs=torch.full((self.B, kc), -7.0, dtype=torch.float32, device=dev),
                       counts=torch.full((self.B, 2), -7, dtype=torch.int32, device=dev),
                       mass=torch.zeros((self.B, 2), dtype=torch.int64, device=dev),
                       cut_ids=torch.full((self.B,), -7, dtype=torch.int32, device=dev))
            out = torch.empty(self.B, dtype=torch.int32, device=dev)
            self.sampler.sample(x["logits"], x["params"], x["u"], hist=x["hist"], hist_len=x["hist_len"], out=out,
                                hint=self.hints[i], debug=dbg)
            torch.cuda.synchronize()
            gp = {k: v.cpu().numpy() for k, v in dbg.items()}
            gp["mass"] = gp["mass"].view(np.uint64)
            gid = out.cpu().numpy()
            cut = lambda a: None if a is None else a[:R]
            o = pyoracle.sample_batch(s["logits"][:R], s["params"][:R], s["u"][:R], hist=cut(s.get("hist")),
                                      hist_len=cut(s.get("hist_len")), mask_table=s.get("mask_table"),
                                      kept_cap=kc, want_post=True, nthreads=nthreads)
            res = o["res"]
            p = s["params"][:R]
            greedy = ((p["flags"] & 1) != 0) | (p["temperature"] <= 0)
            listed = greedy | ((p["top_k"] >= 1) & (p["top_k"] <= 1024) & (p["top_k"] < self.V))
            for b in range(R):
                rep["rows"] += 1
                same = gid[b] == o["ids"][b]
                rep["ids_equal"] += int(same)
                bnd = bool(res["draw_boundary"][b] or res["topp_boundary"][b])
                rep["draw_boundary"] += int(res["draw_boundary"][b])
                rep["topp_boundary"] += int(res["topp_boundary"][b])
                rep["id_disagreements_outside_boundary"] += int(not same and not bnd)
                rep["topk_topp_equal"] += int(gp["counts"][b, 0] == res["n_topk"][b] and gp["counts"][b, 1] == res["n_topp"][b]
                                              and gp["mass"][b, 0] == res["mass_k"][b]
                                              and gp["mass"][b, 1] == res["mass_p"][b]
                                              and gp["cut_ids"][b] == res["cut_id"][b])
                if not listed[b] or o["ids"][b] < 0:
                    continue
                n = min(kc, int(res["n_topk"][b]))
                rep["kept_rows"] += 1
                rep["kept_equal"] += int(np.array_equal(gp["kept_ids"][b, :n], o["kept_ids"][b, :n]))
                m = min(kc, int(res["n_topp"][b]))
                if greedy[b] or m < 1:
                    continue
                rep["prob_rows"] += 1
                rep["probs_bit_equal_oracle"] += int(np.array_equal(gp["kept_probs"][b, :m], o["kept_probs"][b, :m]))
                y = o["post"][b][o["kept_ids"][b, :m]].astype(np.float64)
                e = np.exp(y - y.max())
                pr = e / e.sum()
                err = float(np.max(np.abs(gp["kept_probs"][b, :m].astype(np.float64) - pr) / pr))
                rep["max_rel_prob_err_fp64"] = max(rep["max_rel_prob_err_fp64"], err)
        rep["sets"] = min(n_sets, self.rot)
        rep["rows_per_set"] = R
        return rep

    def cpu_call(self, pyoracle, nthreads):
        def fn(i):
            s = self.sets[i]
            r = pyoracle.sample_batch(s["logits"], s["params"], s["u"], hist=s.get("hist"),
                                      hist_len=s.get("hist_len"), mask_table=s.get("mask_table"),
                                      nthreads=nthreads)
            return r["ids"], s["logits"].shape[0]
        return fn


class SpecVerify:
    """c5: one tgs_spec_verify call per step over B=32 sequences of k=8 drafts."""

    def __init__(self, name, torch, tg, W):
        dev = "cuda:0"
        self.name = name
        self.rot, self.B, self.k, self.V = 2, 32, 8, 128256
        self.sets = [W.config5(B=self.B, k=self.k, V=self.V, seed_offset=i * 1000) for i in range(self.rot)]
        self.sampler = tg.Sampler(device=0, max_batch=self.B, max_vocab=self.V, max_hist=1)
        self.sampler.reserve_spec(self.B, self.k)
        self.d = []
        for s in self.sets:
            self.d.append(dict(
                target=torch.from_numpy(s["target"]).to(dev), draft=torch.from_numpy(s["draft"]).to(dev),
                dtok=torch.from_numpy(s["dtok"]).to(dev), T=torch.from_numpy(s["T"]).to(dev),
                u_acc=torch.from_numpy(s["u_acc"]).to(dev), u_res=torch.from_numpy(s["u_res"]).to(dev),
                n_acc=torch.empty(self.B, dtype=torch.int32, device=dev),
                out=torch.empty(self.B, self.k + 1, dtype=torch.int32, device=dev),
            ))
        self.alg_bytes = W.algorithmic_bytes_per_row("c5", self.V, k=self.k) * self.B
        self.units_per_step = self.B
        self.unit = "rows/s"
        self.metric = "verified sequences/sec, workload c5_spec_verify"
        self.config = {"workload": "c5_spec_verify", "B": 32, "draft_k": 8, "V": 128256, "temperature": 1.0}
        self.dtype = "f32"

    def launch(self, i, stream):
        x = self.d[i % self.rot]
        self.sampler.spec_verify(x["target"], x["draft"], x["dtok"], x["T"], x["u_acc"], x["u_res"],
                                 n_acc=x["n_acc"], out=x["out"], stream=stream)

    def gpu_outputs(self):
        return {i: np.concatenate([self.d[i]["n_acc"].cpu().numpy()[:, None], self.d[i]["out"].cpu().numpy()], 1)
                for i in range(self.rot)}

    def tokens_per_step(self):
        return float(np.mean([(self.d[i]["n_acc"].cpu().numpy() + 1).sum() for i in range(self.rot)]))

    def parity_report(self, pyoracle, nthreads):
        """Accept / reject decisions and emitted tokens of every set against
        the oracle, with the boundary cases (an accept ratio or a draw
        within 1e-6 of its threshold)."""
        rep = dict(sequences=0, n_acc_equal=0, tokens_equal=0, accept_boundary=0, draw_boundary=0,
                   disagreements_outside_boundary=0)
        for i in range(self.rot):
            s = self.sets[i]
            self.launch(i, self.torch_stream())
            g = self.gpu_outputs()[i]
            o = pyoracle.spec_verify_batch(s["target"], s["draft"], s["dtok"], s["T"], s["u_acc"], s["u_res"],
                                           nthreads=nthreads)
            for b in range(self.B):
                rep["sequences"] += 1
                na = g[b, 0] == o["n_acc"][b]
                tok = np.array_equal(g[b, 1:], o["out"][b])
                rep["n_acc_equal"] += int(na)
                rep["tokens_equal"] += int(tok)
                ab, db = int(o["info"]["accept_boundary"][b]), int(o["info"]["draw_boundary"][b])
                rep["accept_boundary"] += ab
                rep["draw_boundary"] += db
                rep["disagreements_outside_boundary"] += int(not (na and tok) and not (ab or db))
        return rep

    def torch_stream(self):
        import torch

        return torch.cuda.current_stream().cuda_stream

    def cpu_call(self, pyoracle, nthreads):
        def fn(i):
            s = self.sets[i]
            r = pyoracle.spec_verify_batch(s["target"], s["draft"], s["dtok"], s["T"], s["u_acc"], s["u_res"],
                                           nthreads=nthreads)
            return np.concatenate([r["n_acc"][:, None], r["out"]], 1), self.B
        return fn


class TokenLogprobs:
    """lp: one tgs_token_logprobs call per step over B=2048 positions of
    V=128256 fp32 logits (generated on the device from a seed); the oracle
    checks the first SAMPLE rows of each set."""

    SAMPLE = 128
    TOL = (1e-4, 1e-6)  # |gpu - oracle| <= atol + rtol |oracle|

    def __init__(self, name, torch, tg, W):
        dev = "cuda:0"
        self.name = name
        self.rot, self.B, self.V = 2, 2048, 128256
        self.sampler = tg.Sampler(device=0, max_batch=64, max_vocab=self.V, max_hist=1)
        self.d, self.host = [], []
        for i in range(self.rot):
            gen = torch.Generator(device=dev).manual_seed(900 + i)
            x = torch.randn(self.B, self.V, device=dev, generator=gen) * 3.0
            tok = torch.randint(0, self.V, (self.B,), device=dev, generator=gen, dtype=torch.int32)
            self.d.append(dict(x=x, tok=tok, out=torch.empty(self.B, dtype=torch.float32, device=dev)))
            self.host.append(dict(x=x[: self.SAMPLE].cpu().numpy(), tok=tok[: self.SAMPLE].cpu().numpy()))
        self.alg_bytes = self.B * (self.V * 4 + 4 + 4)
        self.units_per_step = self.B
        self.unit = "positions/s"
        self.metric = "scored positions/sec (teacher-forced token log-probabilities), workload lp_scoring"
        self.config = {"workload": "lp_scoring", "B": self.B, "V": self.V, "logits": "fp32 N(0, 3^2)"}
        self.dtype = "f32"

    def launch(self, i, stream):
        x = self.d[i % self.rot]
        self.sampler.token_logprobs(x["x"], x["tok"], out=x["out"], stream=stream)

    def gpu_outputs(self):
        return {i: self.d[i]["out"][: self.SAMPLE].cpu().numpy() for i in range(self.rot)}

    def agreement(self, gpu_out, cpu_out):
        atol, rtol = self.TOL
        return float(np.mean([np.mean(np.abs(gpu_out[i] - cpu_out[i]) <= atol + rtol * np.abs(cpu_out[i]))
                              for i in cpu_out]))

    def cpu_call(self, pyoracle, nthreads):
        def fn(i):
            h = self.host[i]
            lp, _ = pyoracle.token_logprobs(h["x"], h["tok"])
            return lp, self.SAMPLE
        return fn


def synthetic_vocab(V, seed=31):
    """A BPE-like byte vocabulary: word pieces of printable ASCII, tag
    pieces, multi-byte UTF-8, and the empty token 0."""
    g = np.random.default_rng(seed)
    pieces = [b"[", b"]", b"POINT", b":", b"none", b",", b"CLICK", b"TYPE", b"SCROLL", b"up", b"KEY", b"+",
              b"OPEN_APP", b" ", b"_", b"-", b"12", b"9"]
    toks = [b""]
    letters = np.frombuffer(b"abcdefghijklmnopqrstuvwxyzABCDEFGHIJ etaoinshr.,", dtype=np.uint8)
    while len(toks) < V:
        r = g.random()
        if r < 0.7:
            n = int(g.integers(1, 13))
            toks.append((b" " if g.random() < 0.4 else b"") + letters[g.integers(0, len(letters), n)].tobytes())
        elif r < 0.9:
            toks.append(b"".join(g.choice(pieces) for _ in range(g.integers(1, 4))))
        else:
            toks.append("".join(chr(int(c)) for c in g.integers(0xC0, 0x2FF, g.integers(1, 4))).encode())
    return toks[:V]


class MaskRows:
    """mask: one tgs_mask_rows_from_dfa call per step building 64 rows (one
    new tool-tag FSM state per sequence of a 64-row batch) over V=151936
    token byte strings; rows rotate over the DFA's states."""

    def __init__(self, name, torch, tg, W):
        from tinygpt_amd import grammar as G

        dev = "cuda:0"
        self.name = name
        self.rot, self.B, self.V = 4, 64, 151936
        self.dfa = G.compile_gbnf(G.PACE_TOOL_TAGS)
        self.toks = synthetic_vocab(self.V)
        off, data = G.token_csr(self.toks)
        self.sampler = tg.Sampler(device=0, max_batch=self.B, max_vocab=self.V, max_hist=1)
        words = (self.V + 31) // 32
        self.sampler.set_mask_table(np.zeros((self.B, words), np.uint32), self.V)
        T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        bc, ct = self.dfa.byte_classes()
        self.byte_class, self.trans = T(bc), T(ct)
        self.complete = T(self.dfa.complete.astype(np.uint8))
        self.off, self.data = T(off), T(data)
        g = np.random.default_rng(5)
        live = np.nonzero(~self.dfa.complete)[0]
        self.states = [g.choice(live, self.B).astype(np.int32) for _ in range(self.rot)]
        self.d_states = [T(s) for s in self.states]
        self.rows = T(np.arange(self.B, dtype=np.int32))
        # token CSR, class map and transition table read once, rows written
        self.alg_bytes = int(off.nbytes + data.nbytes + bc.nbytes + ct.nbytes + self.B * words * 4)
        self.units_per_step = self.B
        self.unit = "rows/s"
        self.metric = "grammar mask rows built/sec (tool-tag DFA, V=151936), workload mask_rows"
        self.config = {"workload": "mask_rows", "B": self.B, "V": self.V, "dfa_states": int(self.dfa.n),
                       "dfa_classes": int(ct.shape[1]),
                       "bound_note": "dependent transition lookups in LDS (one per token byte, 6.3 per token), not HBM"}
        self.dtype = "u8"

    def launch(self, i, stream):
        self.sampler.mask_rows_from_dfa(self.byte_class, self.trans, self.complete, self.off, self.data,
                                        self.d_states[i % self.rot], self.rows, stream=stream)

    def gpu_outputs(self):
        # the table after the last set's call: read back through greedy rows over zero logits
        import torch

        import tinygpt_amd as tg

        dev = "cuda:0"
        i = (self.rot - 1)
        self.launch(i, torch.cuda.current_stream().cuda_stream)
        params = tg.make_params(self.B, temperature=0.0, mask_state=list(range(self.B)))
        post = torch.empty(self.B, self.V, dtype=torch.float32, device=dev)
        self.sampler.sample(torch.zeros(self.B, self.V, device=dev), tg.params_to_device(params, dev),
                            torch.zeros(self.B, device=dev), vocab=self.V, debug={"post_logits": post})
        torch.cuda.synchronize()
        return {i: (post[:4] == 0).cpu().numpy()}

    def cpu_call(self, pyoracle, nthreads):
        def fn(i):
            s = self.states[self.rot - 1][:4]
            w = pyoracle.dfa_mask_rows(self.dfa.trans, self.dfa.complete, self.toks, s)
            bits = np.unpackbits(w.view(np.uint8).reshape(len(s), -1), axis=1, bitorder="little")[:, :self.V]
            return bits.astype(bool), len(s)
        return fn


def json_vocab(V, seed=33):
    """synthetic_vocab with JSON pieces in its last ids: structural runs,
    the schema's keys and enum values, escapes, numbers and every printable
    ASCII byte (a real tokenizer's byte fallback: any document can be
    spelled)."""
    pieces = ['{"', '"}', '":"', '","', '":', '",', '},', '[{', '}]', '[]', '{}', '""', '":{"', '":[', 'true',
              'false', 'null', '\\n', '\\"', '\\u00', '0', '1', '12', '-1', '0.5', 'spokenText', '"spokenText":"',
              'intent', '"intent":"', 'action', 'answer', 'dictate', 'edit', 'out_of_scope', 'clarify',
              'confirm_destructive', 'payload', '"payload":{', 'name', 'args', 'calls', 'text', 'reference', '"}}']
    extra = [p.encode() for p in pieces] + [bytes([c]) for c in range(0x20, 0x7F)]  # every printable byte
    return synthetic_vocab(V - len(extra), seed) + extra


class JsonRows:
    """json: JsonSchemaConstraint.rows_for over 64 snapshots per call (each
    call builds all of them: the constraint forgets its rows first)."""

    SCHEMA = "pace-fm-response-v11"

    def __init__(self, name, torch, tg, W):
        from tinygpt_amd import json_schema as J

        self.name = name
        self.rot, self.B, self.V = 4, 64, 151936
        self.toks = json_vocab(self.V)
        text = open(os.path.join(ROOT, "tests", "golden", "grammars", self.SCHEMA + ".schema.json")).read()
        self.schema_text = text
        self.sampler = tg.Sampler(device=0, max_batch=self.B, max_vocab=self.V, max_hist=1)
        words = (self.V + 31) // 32
        self.sampler.set_mask_table(np.zeros((self.B, words), np.uint32), self.V)
        self.c = J.JsonSchemaConstraint(self.sampler, J.schema_from_json(text), self.toks, eos=self.V - 1,
                                        n_rows=self.B)
        g = np.random.default_rng(11)
        self.sets, self.prefixes = [], []
        while len(self.sets) < self.rot:
            snaps, pre = [], []
            while len(snaps) < self.B:
                s, data = self.c.start(), bytearray()
                for step in range(int(g.integers(2, 200))):  # a random walk of printable bytes
                    ok = [(b, n) for b in range(0x20, 0x7F) if (n := J.JsonSchemaFSM.accept_byte(s, b)) is not None]
                    if not ok:
                        break
                    b, s = ok[int(g.integers(0, len(ok)))]
                    data.append(b)
                snaps.append(s)
                pre.append(bytes(data))
            self.sets.append(snaps)
            self.prefixes.append(pre)
        off, data = __import__("tinygpt_amd.grammar", fromlist=["token_csr"]).token_csr(self.toks)
        self.alg_bytes = int(off.nbytes + data.nbytes + self.B * words * 4)
        self.units_per_step = self.B
        self.unit = "rows/s"
        self.metric = "JSON-schema mask rows built/sec (pace-fm-response-v11, V=151936), workload json_rows"
        self.config = {"workload": "json_rows", "B": self.B, "V": self.V, "schema": self.SCHEMA,
                       "bound_note": "host local DFA (Python) + dependent LDS lookups on the device, not HBM"}
        self.dtype = "u8"

    def launch(self, i, stream):
        self.c.reset()
        self.c.rows_for(self.sets[i % self.rot], stream=stream)

    def gpu_outputs(self):
        import torch

        import tinygpt_amd as tg

        dev = "cuda:0"
        i = self.rot - 1
        self.launch(i, torch.cuda.current_stream().cuda_stream)
        rows = self.c.rows_for(self.sets[i][:4])
        params = tg.make_params(4, temperature=0.0, mask_state=rows.tolist())
        post = torch.empty(4, self.V, dtype=torch.float32, device=dev)
        self.sampler.sample(torch.zeros(4, self.V, device=dev), tg.params_to_device(params, dev),
                            torch.zeros(4, device=dev), vocab=self.V, debug={"post_logits": post})
        torch.cuda.synchronize()
        return {i: (post == 0).cpu().numpy()}

    def cpu_call(self, pyoracle, nthreads):
        import json_fsm

        def fn(i):
            out = []
            for pre in self.prefixes[self.rot - 1][:4]:
                f = json_fsm.FSM(json_fsm.from_json(self.schema_text))
                assert f.accept_bytes(pre)
                out.append(json_fsm.masker_row(f, self.toks, eos=self.V - 1))
            return np.array(out, dtype=bool), 4
        return fn


class JsonDecode:
    """jsondec: one constrained decoding step of 64 sequences per call:
    JsonSchemaConstraint.rows_for, tgs_sample over the masked logits
    (T = 1, top-p 0.95), commit of the 64 ids (a sequence that completes
    samples EOS once and starts a new document)."""

    SCHEMA = "pace-fm-response-v11"

    def __init__(self, name, torch, tg, W):
        from tinygpt_amd import json_schema as J

        dev = "cuda:0"
        self.J, self.tg, self.torch = J, tg, torch
        self.name = name
        self.rot, self.B, self.V = 4, 64, 151936
        self.toks = json_vocab(self.V)
        self.eos = 0  # the empty token: never allowed but as EOS
        text = open(os.path.join(ROOT, "tests", "golden", "grammars", self.SCHEMA + ".schema.json")).read()
        self.schema_text = text
        self.sampler = tg.Sampler(device=0, max_batch=self.B, max_vocab=self.V, max_hist=1)
        n_rows = 4096
        self.sampler.set_mask_table(np.zeros((n_rows, (self.V + 31) // 32), np.uint32), self.V)
        self.c = J.JsonSchemaConstraint(self.sampler, J.schema_from_json(text), self.toks, eos=self.eos,
                                        n_rows=n_rows)
        g = np.random.default_rng(12)
        # closing pieces likelier, so documents finish; tokens that are not UTF-8 never sampled
        bias = np.zeros(self.V, np.float32)
        for i, t in enumerate(self.toks):
            try:
                t.decode("utf-8")
            except UnicodeDecodeError:
                bias[i] = -np.inf
                continue
            if b'"' in t or b"}" in t:
                bias[i] = 3.0
        self.d_logits = [torch.from_numpy(W.normal_f32(g, (self.B, self.V), 3.0) + bias).to(dev)
                         for _ in range(self.rot)]
        self.d_u = [torch.from_numpy(W.uniforms(g, self.B)).to(dev) for _ in range(self.rot)]
        self.params = tg.make_params(self.B, temperature=1.0, top_p=0.95)
        self.out = torch.empty(self.B, dtype=torch.int32, device=dev)
        self.snaps = [self.c.start()] * self.B
        self.docs = [bytearray() for _ in range(self.B)]
        self.completed = 0
        self.stuck = 0  # documents no token could continue (id -1, nothing allowed)
        self.checks = []  # (prefix, id) pairs kept for the parity check
        # per step, as the reference's per-token trace (InferenceTracer.addToken,
        # native-mac/Sources/TinyGPTServe/InferenceTrace.swift:40-134) splits a
        # token's time: the constraint (automaton snapshots interned as rows,
        # new rows built on the device), the sampling call (parameters up, ids
        # back) and the commit of the sampled ids to the automaton
        self.trace = []
        self.alg_bytes = self.B * self.V * 4
        self.units_per_step = self.B
        self.unit = "tokens/s"
        self.metric = "JSON-schema constrained decode tokens/sec (64 sequences, pace-fm-response-v11, V=151936)"
        self.config = {"workload": "jsondec", "B": self.B, "V": self.V, "schema": self.SCHEMA, "temperature": 1.0,
                       "top_p": 0.95, "bound_note": "host automaton and row interning per step; the sampling call "
                                                    "is the C3-style masked top-p kernel"}
        self.dtype = "f32"

    def launch(self, i, stream):
        tg = self.tg
        st = self.torch.cuda.ExternalStream(stream)
        t0 = time.perf_counter()
        built0 = self.c.built
        try:
            rows = self.c.rows_for(self.snaps, stream=stream)
        except RuntimeError:  # the constraint's rows are used up: start over
            self.c.reset()
            rows = self.c.rows_for(self.snaps, stream=stream)
        st.synchronize()
        t1 = time.perf_counter()
        self.params["mask_state"] = rows
        pd = tg.params_to_device(self.params, "cuda:0")
        self.sampler.sample(self.d_logits[i % self.rot], pd, self.d_u[i % self.rot], out=self.out, stream=stream,
                            hint=tg.batch_hint(self.params, self.V))
        with self.torch.cuda.stream(st):
            ids = self.out.cpu().numpy()
        t2 = time.perf_counter()
        self._commit(ids)
        t3 = time.perf_counter()
        self.trace.append((len(self.trace), (t1 - t0) * 1e3, (t2 - t1) * 1e3, (t3 - t2) * 1e3,
                           self.c.built - built0))

    def trace_summary(self, first=8):
        """Per-step times in ms: mean / p50 / p90 of each part over the
        steps, and the first steps as recorded."""
        if not self.trace:
            return None
        a = np.array([t[1:4] for t in self.trace], np.float64)
        out = {"steps": len(self.trace), "unit": "ms per step of 64 tokens"}
        for j, name in enumerate(("constraint", "sample", "commit")):
            out[name] = {"mean": round(float(a[:, j].mean()), 3), "p50": round(float(np.percentile(a[:, j], 50)), 3),
                         "p90": round(float(np.percentile(a[:, j], 90)), 3)}
        out["rows_built_per_step"] = round(float(np.mean([t[4] for t in self.trace])), 2)
        out["first_steps"] = [{"index": t[0], "constraint_ms": round(t[1], 3), "sample_ms": round(t[2], 3),
                               "commit_ms": round(t[3], 3), "rows_built": t[4]} for t in self.trace[:first]]
        return out

    def _commit(self, ids):
        for b in range(self.B):
            t = int(ids[b])
            if t < 0:  # no token of this vocabulary continues the document: start a new one
                self.snaps[b], self.docs[b] = self.c.start(), bytearray()
                self.stuck += 1
                continue
            if len(self.checks) < 8 and b < 2:
                self.checks.append((bytes(self.docs[b]), t))
            if self.J.JsonSchemaFSM.is_complete(self.snaps[b]):
                if t != self.eos:
                    raise RuntimeError(f"a complete sequence sampled {t}, not EOS")
                self.snaps[b], self.docs[b] = self.c.start(), bytearray()
                self.completed += 1
                continue
            n = self.c.commit(self.snaps[b], t)
            if n is None:
                raise RuntimeError(f"sampled token {t} rejected by the automaton")
            self.snaps[b] = n
            self.docs[b] += self.toks[t]

    def gpu_outputs(self):
        return {0: np.array([t for _, t in self.checks], np.int64)}

    def cpu_call(self, pyoracle, nthreads):
        import json_fsm

        def fn(i):
            ok = []
            for pre, t in self.checks:
                f = json_fsm.FSM(json_fsm.from_json(self.schema_text))
                assert f.accept_bytes(pre)
                row = json_fsm.masker_row(f, self.toks, eos=self.eos)
                ok.append(t if row[t] else -1)  # the sampled id when the reference's masker allows it
            return np.array(ok, np.int64), len(self.checks)
        return fn


class FloorRead:
    """read: the plain-read floor under the C2 headline.  The same 16
    rotating 64 x 128256 fp32 sets, read by libtgs_floor.so with the fused
    top_k <= 64 kernel's grid and load pattern (4 chunks per row, 512
    threads, 16 non-temporal 16-byte loads per thread at entry) and nothing
    computed but each chunk's maximum: the time the sampling chain adds its
    work to.  Not part of the sampler; no CPU baseline."""

    def __init__(self, name, torch, tg, W):
        import ctypes as C

        dev = "cuda:0"
        self.rot, self.B, self.V, self.S = 16, 64, 128256, 4
        lib = C.CDLL(os.path.join(ROOT, "tinygpt_amd", "libtgs_floor.so"))
        lib.tgs_floor_read.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_longlong, C.c_int, C.c_void_p, C.c_void_p]
        lib.tgs_floor_read.restype = C.c_int
        self.lib, self.C = lib, C
        self.x = [torch.from_numpy(W.config2(B=self.B, V=self.V, seed_offset=i * 1000)["logits"]).to(dev)
                  for i in range(self.rot)]
        self.out = torch.empty(self.B * self.S, dtype=torch.float32, device=dev)
        self.config = {"workload": "read_floor_c2", "B": self.B, "V": self.V, "chunks_per_row": self.S,
                       "threads_per_chunk": 512, "loads": "16 non-temporal 16-byte loads per thread"}
        self.dtype = "f32"
        self.alg_bytes = 4 * self.V * self.B
        self.units_per_step = self.B
        self.unit = "rows/s"
        self.metric = "rows/sec read by a plain read of the C2 logits (the floor under the headline)"

    def launch(self, i, stream):
        C = self.C
        rc = self.lib.tgs_floor_read(C.c_void_p(self.x[i % self.rot].data_ptr()), self.B, self.V, self.V, self.S,
                                     C.c_void_p(self.out.data_ptr()), C.c_void_p(stream))
        if rc != 0:
            raise RuntimeError(f"tgs_floor_read: {rc}")

    def gpu_outputs(self):
        return {}


def cpu_baseline(wl, seconds):
    """The oracle (C restatement of the reference sampler) on this host:
    units/s with all host threads (up to 16) and with one thread."""
    pyoracle = oracle_mod()
    nthr = cpu_threads()
    if isinstance(wl, JsonDecode):  # the reference's masker on the checked steps, one thread
        rate, units, outs = timed_loop(wl.cpu_call(pyoracle, 1), 1, seconds)
        return dict(value=round(rate, 3), unit="masked rows/s", cores=1, kind="port",
                    host_cpu_count=os.cpu_count(), host_cpu_model=cpu_model(),
                    sample=f"{units} rows: the oracle's clone-and-replay of LogitsMasker.mask over V={wl.V} for "
                           f"sampled steps of two sequences, 1 thread (the reference's masking cost per token)"), outs
    if isinstance(wl, JsonRows):  # the reference's clone-and-replay masker, one thread
        rate, units, outs = timed_loop(wl.cpu_call(pyoracle, 1), 1, seconds)
        outs = {wl.rot - 1: outs[0]}
        return dict(value=round(rate, 3), unit=wl.unit, cores=1, kind="port",
                    host_cpu_count=os.cpu_count(), host_cpu_model=cpu_model(),
                    sample=f"{units} rows (4 snapshots of the last set, V={wl.V}, the oracle's per-token "
                           f"clone-and-replay of LogitsMasker.mask in Python) on 1 thread"), outs
    rate_n, units_n, outs = timed_loop(wl.cpu_call(pyoracle, nthr), wl.rot, seconds * 0.6)
    rate_1, units_1, _ = timed_loop(wl.cpu_call(pyoracle, 1), wl.rot, seconds * 0.4)
    if isinstance(wl, MaskRows):  # vectorised numpy DFA replay, one thread
        rate, units, outs = timed_loop(wl.cpu_call(pyoracle, 1), 1, seconds)
        outs = {wl.rot - 1: outs[0]}
        return dict(value=round(rate, 2), unit=wl.unit, cores=1, kind="port",
                    host_cpu_count=os.cpu_count(), host_cpu_model=cpu_model(),
                    sample=f"{units} rows (4 states of the last set, V={wl.V}, numpy vectorised byte replay) "
                           f"on 1 thread"), outs
    if isinstance(wl, TokenLogprobs):  # numpy, one thread
        rate, units, outs = timed_loop(wl.cpu_call(pyoracle, 1), wl.rot, seconds)
        return dict(value=round(rate, 2), unit=wl.unit, cores=1, kind="port",
                    host_cpu_count=os.cpu_count(), host_cpu_model=cpu_model(),
                    sample=f"{units} positions of lp_scoring (the first {wl.SAMPLE} rows of each of {wl.rot} "
                           f"seeded sets, float64 numpy log-softmax) on 1 thread"), outs
    return dict(
        value=round(rate_n, 2), unit=wl.unit, cores=nthr, kind="port",
        sample=f"{units_n} rows of {wl.config['workload']} (batches of {wl.B} cycling over {wl.rot} seeded sets) "
               f"on {nthr} threads; 1 thread: {round(rate_1, 2)} {wl.unit} over {units_1} rows",
        single_thread_value=round(rate_1, 2),
        host_cpu_count=os.cpu_count(), host_cpu_model=cpu_model(),
        threads_note="every core this process may run on, at most 16 (a one-GPU box's share of the host)",
    ), outs


def calibrate_copy(torch, mib, reps=8):
    """Plain copy of a known size, for scaling HBM byte counters."""
    n = mib << 20
    src = torch.empty(n // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / reps
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "reps": reps,
                      "ms_per_copy": round(ms, 4), "GBps": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)


TRAFFIC_FILES = {"c2": "k64_kernel_c2_traffic.json", "c3": "c3_grammar_traffic.json",
                 "c4": "c4_large_batch_traffic.json", "c5": "c5_spec_verify_traffic.json"}
TRAFFIC_FILES["lp"] = "lp_scoring_traffic.json"
TRAFFIC_FILES["c2m"] = "k64_kernel_c2m_traffic.json"
TRAFFIC_FILES["json"] = "json_rows_traffic.json"
TRAFFIC_FILES["mask"] = "mask_rows_traffic.json"
TRAFFIC_FILES["read"] = "read_floor_c2_traffic.json"
KERNELS = {"read": "floor_read_kernel (libtgs_floor.so)", "c1": "k64_kernel<float> (one-wave)", "c2": "k64_kernel<float>", "c2m": "k64_kernel<float> (mask variant)",
           "c3": "topp_kernel<float, true>",
           "c4": "topk_kernel<bf16, 20>",
           "c5": "spec_block_kernel + spec_decide_kernel + spec_mass_kernel + spec_draw_kernel (one call)",
           "lp": "lp::chunk_kernel<float>", "mask": "maskb::prep_image + maskb::build_lds (one call)",
           "json": "host local DFA + maskb kernels (one call)",
           "jsondec": "host automaton + mask rows + topp_kernel per step"}


def time_calls(torch, wl, stream, steps, eager):
    """GPU time per call of `steps` calls of wl, between two events on the
    launch stream.  Graph replay: the timed calls are one captured graph of
    `per` calls (cycling over the rotating input sets), replayed `reps` times;
    per = steps up to 4096 calls, so that a short run launches one graph.
    Returns (ms per call, the graph or None)."""
    ROT = wl.rot
    per = steps if steps <= 4096 else ROT * max(1, 4096 // ROT)
    reps, rem = divmod(steps, per)

    def capture(n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
            for i in range(n):
                wl.launch(i, stream.cuda_stream)
        torch.cuda.synchronize()
        return g

    graph = graph_rem = None
    if not eager:
        graph = capture(per) if reps else None
        graph_rem = capture(rem) if rem else None
        for g in (graph, graph_rem):
            if g is not None:
                g.replay()
        torch.cuda.synchronize()

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        # The same calls, untimed, ahead of the start event keep the GPU busy
        # while the host submits the timed graph, so the timed region holds
        # the K calls alone (in a decode loop the sampler is queued behind
        # the model's forward pass the same way).
        if not eager:
            for g in (graph, graph_rem):
                if g is not None:
                    g.replay()
        else:
            torch.cuda._sleep(200000)
        ev0.record(stream)
        if not eager:
            for _ in range(reps):
                graph.replay()
            if graph_rem is not None:
                graph_rem.replay()
        else:
            for i in range(steps):
                wl.launch(i, stream.cuda_stream)
        ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps, graph


def sub_line(torch, wl, stream, steps, args, name):
    """One more workload timed like the main line, reported as a sub-object."""
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            wl.launch(i, stream.cuda_stream)
    torch.cuda.synchronize()
    ms, graph = time_calls(torch, wl, stream, steps, args.eager)
    achieved = wl.alg_bytes / (ms * 1e-3) / 1e9
    return {"workload": wl.config["workload"], "us_per_call": round(ms * 1e3, 3),
            "value": round(wl.units_per_step / (ms * 1e-3), 1), "unit": wl.unit,
            "timing": "graph replay" if graph is not None else "eager", "steps": steps,
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "alg_bytes_per_launch": wl.alg_bytes,
                         "kernel": KERNELS[name]}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build runs on a "
              "single GPU; the sampler is row-parallel and would shard by batch rows with "
              "no exchange between GPUs", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.calibrate_copy:
        calibrate_copy(torch, args.calibrate_copy)
        return

    import tinygpt_amd as tg
    from tinygpt_amd import workloads as W

    if args.workload == "c5":
        wl = SpecVerify(args.workload, torch, tg, W)
    elif args.workload == "lp":
        wl = TokenLogprobs(args.workload, torch, tg, W)
    elif args.workload == "mask":
        wl = MaskRows(args.workload, torch, tg, W)
    elif args.workload == "json":
        wl = JsonRows(args.workload, torch, tg, W)
        args.eager = True  # the host builds each call's automaton: no graph
    elif args.workload == "jsondec":
        wl = JsonDecode(args.workload, torch, tg, W)
        args.eager = True
    elif args.workload == "read":
        wl = FloorRead(args.workload, torch, tg, W)
        args.no_cpu = True  # a measurement floor, not a sampler: nothing to compare
    else:
        wl = Sampling(args.workload, torch, tg, W)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device="cuda:0")  # default priority
    ROT = wl.rot

    with torch.cuda.stream(stream):
        for i in range(min(args.warmup, 4) if isinstance(wl, (JsonRows, JsonDecode)) else args.warmup):
            wl.launch(i, stream.cuda_stream)
    torch.cuda.synchronize()

    steps = max(1, args.steps)
    if isinstance(wl, (JsonRows, JsonDecode)):
        steps = min(steps, 64 if isinstance(wl, JsonRows) else 200)  # host work in every call
    if isinstance(wl, JsonDecode):
        wl.trace = []  # the timed steps only
    ms_per_step, graph = time_calls(torch, wl, stream, steps, args.eager)
    trace = wl.trace_summary() if isinstance(wl, JsonDecode) else None

    # per-call distribution: eager calls, each between two events
    n_calls = 16 if isinstance(wl, (JsonRows, JsonDecode)) else 256
    e_start = [torch.cuda.Event(enable_timing=True) for _ in range(n_calls)]
    e_end = [torch.cuda.Event(enable_timing=True) for _ in range(n_calls)]
    with torch.cuda.stream(stream):
        for i in range(n_calls):
            e_start[i].record(stream)
            wl.launch(i, stream.cuda_stream)
            e_end[i].record(stream)
    torch.cuda.synchronize()
    per_call = np.array([a.elapsed_time(b) * 1e3 for a, b in zip(e_start, e_end)])
    per_call_us = {"p10": round(float(np.percentile(per_call, 10)), 2),
                   "p50": round(float(np.percentile(per_call, 50)), 2),
                   "p90": round(float(np.percentile(per_call, 90)), 2), "calls": n_calls,
                   "mode": "eager launches, HIP events around each call on the launch stream"}

    # parity of the timed outputs against the oracle (same inputs)
    gpu_out = wl.gpu_outputs()
    cpu = None
    agreement = None
    parity = None
    if not args.no_cpu:
        cpu, cpu_out = cpu_baseline(wl, args.cpu_seconds)
        if isinstance(wl, TokenLogprobs):
            agreement = wl.agreement(gpu_out, cpu_out)
        else:
            agreement = float(np.mean([np.mean(gpu_out[i] == cpu_out[i]) for i in cpu_out]))
        if agreement != 1.0:
            print("WARNING: GPU outputs differ from the oracle", file=sys.stderr)
        if hasattr(wl, "parity_report"):
            parity = wl.parity_report(oracle_mod(), cpu_threads())

    achieved = wl.alg_bytes / (ms_per_step * 1e-3) / 1e9
    units_per_s = wl.units_per_step / (ms_per_step * 1e-3)
    traffic = None
    tf = TRAFFIC_FILES.get(args.workload)
    if tf and os.path.exists(os.path.join(ROOT, "profiles", tf)):
        try:
            traffic = json.load(open(os.path.join(ROOT, "profiles", tf))).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None
    cfg = dict(wl.config)
    cfg["rotating_sets"] = ROT
    cfg["timing"] = "graph replay" if graph is not None else "eager"
    line = {
        "metric": wl.metric,
        "value": round(units_per_s, 1),
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": "synthetic",
        "config": cfg,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "alg_bytes_per_launch": wl.alg_bytes, "kernel": KERNELS[args.workload]},
        "cpu_baseline": cpu,
        "id_agreement": agreement,
        "parity": parity,
        "per_call_us": per_call_us,
    }
    if args.workload == "c2" and not args.no_c2m:
        # the same chain with the grammar mask stage, and the plain read of
        # the same logits: both timed like the headline, on the same stream
        line["c2m"] = sub_line(torch, Sampling("c2m", torch, tg, W), stream, steps, args, "c2m")
        if os.path.exists(os.path.join(ROOT, "tinygpt_amd", "libtgs_floor.so")):
            line["read_floor"] = sub_line(torch, FloorRead("read", torch, tg, W), stream, steps, args, "read")
    if isinstance(wl, SpecVerify):
        line["tokens_per_s"] = round(wl.tokens_per_step() / (ms_per_step * 1e-3), 1)
    if isinstance(wl, JsonDecode):
        line["trace"] = trace
        line["documents_completed"] = wl.completed
        line["documents_stuck"] = wl.stuck
        line["mask_rows_built"] = wl.c.built
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
