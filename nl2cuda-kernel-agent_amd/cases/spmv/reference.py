"""PyTorch reference of CSR SpMM / SpMV and the input generators.

``reference_forward`` is the reference's cases/spmv/reference.py:8-23 (row
ids by repeat_interleave, vals * X[col_idx], index_add_ into zeros);
autograd gives dvals and dX.  Inputs are drawn on the host CPU generator and
moved to ``device`` so both sides see identical tensors.

``zipf_row_lengths`` / ``make_zipf_inputs`` are the acceptance workload's
deterministic recipe (numpy Generator(seed)):
  1. raw = min(zipf(1.5, M), 4096);
  2. scaled = raw * (16 M / sum(raw)); lens = clip(floor(scaled), 1, min(4096, K));
  3. while sum(lens) != 16 M: if short, +1 to the rows with the largest
     fractional part of `scaled` (ties: lower row first) that can still grow;
     if over, -1 to the longest rows (ties: lower row first) above 1;
  4. columns: per row `len` distinct values ~ U[0, K), sorted ascending
     (drawn for all rows at once, duplicates within a row redrawn until none
     are left);
  5. vals, x, dy ~ N(0, 1) from torch.Generator(seed) on the CPU.
"""

import numpy as np
import torch

from cases.spmv import config


def reference_forward(inputs, params):
    del params
    row_ptr = inputs["row_ptr"]
    col_idx = inputs["col_idx"]
    vals = inputs["vals"]
    X = inputs["X"]
    row_counts = row_ptr[1:] - row_ptr[:-1]
    row_idx = torch.repeat_interleave(
        torch.arange(row_counts.shape[0], device=row_ptr.device), row_counts)
    contributions = vals.unsqueeze(1) * X.index_select(0, col_idx)
    output = torch.zeros((row_counts.shape[0], X.shape[1]), dtype=X.dtype, device=X.device)
    return output.index_add_(0, row_idx, contributions)


def make_inputs_for(m, k, d, nnz_per_row):
    """The reference's uniform generator (reference.py:26-51): every row has
    nnz_per_row columns drawn with replacement, int64 indices."""

    def make_inputs(seed, dtype, device, requires_grad=False):
        g = torch.Generator(device="cpu").manual_seed(seed)
        nnz = m * nnz_per_row
        row_ptr = torch.arange(m + 1, dtype=torch.int64) * nnz_per_row
        col_idx = torch.randint(0, k, (nnz,), dtype=torch.int64, generator=g)
        vals = torch.randn(nnz, generator=g).to(dtype)
        X = torch.randn(k, d, generator=g).to(dtype)
        out = {"row_ptr": row_ptr.to(device), "col_idx": col_idx.to(device),
               "vals": vals.to(device), "X": X.to(device)}
        if requires_grad:
            out["vals"].requires_grad_(True)
            out["X"].requires_grad_(True)
        return out

    return make_inputs


def zipf_row_lengths(m, k, seed, s=config.ZIPF_S, max_len=config.MAX_ROW,
                     mean=config.BASELINE_MEAN):
    rng = np.random.default_rng(seed)
    cap = min(max_len, k)
    raw = np.minimum(rng.zipf(s, m), max_len).astype(np.float64)
    target = mean * m
    scaled = raw * (target / raw.sum())
    lens = np.clip(np.floor(scaled), 1, cap).astype(np.int64)
    frac = scaled - np.floor(scaled)
    idx = np.arange(m)
    while lens.sum() != target:
        diff = int(target - lens.sum())
        if diff > 0:
            order = np.lexsort((idx, -frac))
            cand = order[lens[order] < cap]
            if cand.size == 0:
                raise ValueError("cannot reach the target nnz")
            lens[cand[:diff]] += 1
        else:
            order = np.lexsort((idx, -lens))
            cand = order[lens[order] > 1]
            if cand.size == 0:
                raise ValueError("cannot reach the target nnz")
            lens[cand[:-diff]] -= 1
    return lens


def sorted_unique_columns(lens, k, seed):
    rng = np.random.default_rng(seed + 1)
    m = lens.shape[0]
    row_of = np.repeat(np.arange(m, dtype=np.int64), lens)
    key = row_of * k + rng.integers(0, k, row_of.shape[0])
    key.sort()
    while True:
        dup = np.flatnonzero(key[1:] == key[:-1]) + 1
        if dup.size == 0:
            break
        key[dup] = row_of[dup] * k + rng.integers(0, k, dup.size)
        key.sort()
    return key - row_of * k


def make_zipf_inputs(m, k, d, seed, index_dtype=torch.int32):
    lens = zipf_row_lengths(m, k, seed)
    row_ptr = np.zeros(m + 1, dtype=np.int64)
    np.cumsum(lens, out=row_ptr[1:])
    cols = sorted_unique_columns(lens, k, seed)
    g = torch.Generator(device="cpu").manual_seed(seed)
    nnz = int(row_ptr[-1])
    vals = torch.randn(nnz, generator=g)
    X = torch.randn(k, d, generator=g)
    return {"row_ptr": torch.from_numpy(row_ptr).to(index_dtype),
            "col_idx": torch.from_numpy(cols).to(index_dtype), "vals": vals, "X": X}


def make_zipf_inputs_for(m, k, d, index_dtype=torch.int32):
    cache = {}

    def make_inputs(seed, dtype, device, requires_grad=False):
        if seed not in cache:
            cache.clear()
            cache[seed] = make_zipf_inputs(m, k, d, seed, index_dtype)
        out = {key: v.to(device) for key, v in cache[seed].items()}
        out["vals"] = out["vals"].to(dtype)
        out["X"] = out["X"].to(dtype)
        if requires_grad:
            out["vals"].requires_grad_(True)
            out["X"].requires_grad_(True)
        return out

    return make_inputs


make_inputs = make_inputs_for(config.M, config.K, config.D, config.NNZ_PER_ROW)
