"""Runs tgs_sample through the CPU simulation of the kernels (built by the
Makefile beside this file, under AddressSanitizer) and returns the same
outputs as the GPU harness.  TEST INFRASTRUCTURE ONLY: a debugging aid for
kernel memory errors, never part of the product path."""
from __future__ import annotations

import fcntl
import os
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.environ.get("TGS_SIM_BIN", os.path.join(HERE, "build", "run_case"))


def build():
    # One build at a time across test worker processes; the Makefile writes
    # each binary under a temporary name and renames it into place, so a
    # worker still running the previous binary is not disturbed.
    os.makedirs(os.path.join(HERE, "build"), exist_ok=True)
    with open(os.path.join(HERE, "build", ".lock"), "w") as lk:
        fcntl.flock(lk, fcntl.LOCK_EX)
        subprocess.run(["make", "-s", f"-j{min(8, os.cpu_count() or 1)}", "-C", HERE], check=True)


def _san_env():
    """Sanitizer options of every simulated run.  Device memory is never
    zeroed on the GPU, so every allocation is filled with a poison byte: a
    kernel that reads memory nothing wrote then sees garbage here too."""
    return {"ASAN_OPTIONS": os.environ.get(
                "ASAN_OPTIONS", "detect_leaks=0:abort_on_error=0:max_malloc_fill_size=2147483647:malloc_fill_byte=190"),
            "UBSAN_OPTIONS": os.environ.get("UBSAN_OPTIONS", "halt_on_error=1:print_stacktrace=1")}


def run_sample(logits, params, u, hist=None, hist_len=None, mask_table=None, V=None, kept_cap=64,
               post=True, hint=None, split=None, timeout=600, noalloc=False, concurrent=False, repeat=1,
               env_extra=None):
    """hint: None (general kernel) or an int max_top_k.  noalloc: through
    tgs_sample_noalloc (static workspace) instead of a handle.  concurrent:
    every workgroup of a launch runs at once (the split k64 kernel's chunks
    then exchange their row-wide bound; only launches of that kernel may run
    so).  repeat: that many calls, each of whose ids must equal the first's."""
    B = logits.shape[0]
    V = logits.shape[1] if V is None else V
    dtype = 1 if logits.dtype == np.uint16 else 0
    hist_cap = 0 if hist is None else hist.shape[1]
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as d:
        np.ascontiguousarray(logits).tofile(os.path.join(d, "logits.bin"))
        np.ascontiguousarray(params).tofile(os.path.join(d, "params.bin"))
        np.asarray(u, np.float32).tofile(os.path.join(d, "u.bin"))
        if hist is not None:
            np.ascontiguousarray(hist, np.int32).tofile(os.path.join(d, "hist.bin"))
        if hist_len is not None:
            np.ascontiguousarray(hist_len, np.int32).tofile(os.path.join(d, "hist_len.bin"))
        n_states = 0
        if mask_table is not None:
            n_states = mask_table.shape[0]
            np.ascontiguousarray(mask_table, np.uint32).tofile(os.path.join(d, "mask.bin"))
        with open(os.path.join(d, "meta.txt"), "w") as f:
            f.write(f"{B} {V} {logits.shape[1]} {dtype} {hist_cap} {int(hist_len is not None)} {n_states} "
                    f"{-1 if hint is None else int(hint)} {kept_cap} {int(bool(post))} "
                    f"{int(getattr(hint, 'min_top_k', 0))}\n")
        env = dict(os.environ)
        if split is not None:
            env["TGS_SPLIT"] = str(split)
        if noalloc:
            env["TGS_SIM_NOALLOC"] = "1"
        if concurrent:
            env["TGS_SIM_CONCURRENT"] = "1"
        else:
            # workgroups run one after another here: a chunk's partners have
            # not run yet when it polls their keys, so it gives up at once
            # and keeps its own bound (the row's last chunk sees every key)
            env.setdefault("TGS_KEY_SPINS", "1")
        if repeat > 1:
            env["TGS_SIM_REPEAT"] = str(repeat)
        if env_extra:
            env.update(env_extra)
        env.update(_san_env())
        env["TGS_SIM_TRACE"] = "1"
        p = subprocess.run([BIN, "sample", d], capture_output=True, text=True, env=env, timeout=timeout)
        launches = [tuple(int(f.split("=")[1]) for f in l.split()[1:3])
                    for l in p.stderr.splitlines() if l.startswith("launch grid=")]
        err = "\n".join(l for l in p.stderr.splitlines() if not l.startswith("launch grid="))
        if err.strip():
            print(err[-12000:])
        if p.returncode != 0:
            raise RuntimeError(f"run_case exit {p.returncode}\n{p.stdout[-4000:]}\n{p.stderr[-12000:]}")
        rd = lambda n, dt: np.fromfile(os.path.join(d, n), dt)
        r = dict(ids=rd("out_ids.bin", np.int32),
                 kept_ids=rd("out_kept_ids.bin", np.int32).reshape(B, kept_cap),
                 kept_probs=rd("out_kept_probs.bin", np.float32).reshape(B, kept_cap),
                 counts=rd("out_counts.bin", np.int32).reshape(B, 2),
                 mass=rd("out_mass.bin", np.uint64).reshape(B, 2),
                 cut_ids=rd("out_cut.bin", np.int32),
                 post_logits=rd("out_post.bin", np.float32).reshape(B, V) if post else None)
        r["launches"] = launches  # (grid, block) of every kernel launch, in order
        r["stdout"] = p.stdout
        return r


def run_maskbuild(byte_class, trans, complete, tok_off, tok_bytes, states, rows, n_rows, eos=-1, timeout=600):
    """tgs_mask_rows_from_dfa through the simulation (trans [n_dfa, n_cls]),
    read back as the post_logits of greedy rows over zero logits: float32
    [n_rows, V]."""
    V = len(tok_off) - 1
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as d:
        for name, arr, dt in (("byte_class", byte_class, np.uint8), ("trans", trans, np.int32),
                              ("complete", complete, np.uint8), ("tok_off", tok_off, np.int32),
                              ("tok_bytes", tok_bytes, np.uint8), ("states", states, np.int32), ("rows", rows, np.int32)):
            np.ascontiguousarray(arr, dt).tofile(os.path.join(d, name + ".bin"))
        with open(os.path.join(d, "meta.txt"), "w") as f:
            f.write(f"{trans.shape[0]} {trans.shape[1]} {V} {len(states)} {eos} {n_rows}\n")
        r = subprocess.run([BIN, "maskbuild", d], capture_output=True, text=True, timeout=timeout,
                           env={**os.environ, **_san_env()})
        if r.returncode != 0:
            raise RuntimeError(f"simulation failed ({r.returncode}):\n{r.stdout}\n{r.stderr}")
        return np.fromfile(os.path.join(d, "out_post.bin"), np.float32).reshape(n_rows, V)


def run_logprob(logits, tokens, V=None, timeout=600):
    """tgs_token_logprobs through the simulation: (logprob [B], lse [B]).
    logits [B, row_stride] float32 or bf16 bits (uint16); V <= row_stride."""
    logits = np.ascontiguousarray(logits)
    B, stride = logits.shape
    V = stride if V is None else V
    dtype = 1 if logits.dtype == np.uint16 else 0
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as d:
        logits.tofile(os.path.join(d, "logits.bin"))
        np.ascontiguousarray(tokens, np.int32).tofile(os.path.join(d, "tokens.bin"))
        with open(os.path.join(d, "meta.txt"), "w") as f:
            f.write(f"{B} {V} {stride} {dtype}\n")
        r = subprocess.run([BIN, "logprob", d], capture_output=True, text=True, timeout=timeout,
                           env={**os.environ, **_san_env()})
        if r.returncode != 0:
            raise RuntimeError(f"simulation failed ({r.returncode}):\n{r.stdout}\n{r.stderr}")
        return (np.fromfile(os.path.join(d, "out_lp.bin"), np.float32),
                np.fromfile(os.path.join(d, "out_lse.bin"), np.float32))


def run_spec(target, draft, dtok, T, u_acc, u_res, timeout=600):
    """tgs_spec_verify through the simulation: (n_acc [B], out [B, k+1])."""
    target = np.ascontiguousarray(target)
    B, k1, V = target.shape
    k = k1 - 1
    dtype = 1 if target.dtype == np.uint16 else 0
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as d:
        target.tofile(os.path.join(d, "target.bin"))
        np.ascontiguousarray(draft).tofile(os.path.join(d, "draft.bin"))
        np.ascontiguousarray(dtok, np.int32).tofile(os.path.join(d, "dtok.bin"))
        np.ascontiguousarray(T, np.float32).tofile(os.path.join(d, "T.bin"))
        np.ascontiguousarray(u_acc, np.float32).tofile(os.path.join(d, "u_acc.bin"))
        np.ascontiguousarray(u_res, np.float32).tofile(os.path.join(d, "u_res.bin"))
        with open(os.path.join(d, "meta.txt"), "w") as f:
            f.write(f"{B} {k} {V} {dtype}\n")
        r = subprocess.run([BIN, "spec", d], capture_output=True, text=True, timeout=timeout,
                           env={**os.environ, **_san_env()})
        if r.returncode != 0:
            raise RuntimeError(f"simulation failed ({r.returncode}):\n{r.stdout}\n{r.stderr}")
        n_acc = np.fromfile(os.path.join(d, "out_nacc.bin"), np.int32)
        out = np.fromfile(os.path.join(d, "out_spec.bin"), np.int32).reshape(B, k + 1)
        return n_acc, out
