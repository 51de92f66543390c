"""The frozen projections' plain fp16 GEMMs through qlora_gemm (rocBLAS, Tensile kernels) with a
solution measured per weight shape and token-count bucket.

y = x W^T and dX = dY W (engine.py:1082-1316) are torch matmuls in the reference, i.e. whatever
kernel the library's size heuristic picks. At this step's sizes (M = a few thousand tokens) the
heuristic leaves 20-30 % on the table for the widest projections (gate|up: 0.93 -> 1.15 PFLOP/s
forward, 0.65 -> 0.83 backward on MI355X). The tuner times every solution rocBLAS offers for a
shape once, keeps the fastest few as candidates, and then, per bucket of BUCKET tokens, the
fastest candidate (torch's own matmul is one of them). Results are bit-for-bit those of an fp16
GEMM with fp32 accumulation; only the summation order differs between solutions.
"""

import ctypes
import time

import torch

from . import _lib
from .ops import _need, _ptr, _stream

BUCKET = 256
TORCH = -1       # candidate: torch's matmul
DEFAULT = 0      # candidate: rocBLAS's own choice
NT, NN = 0, 1    # op: C = A B^T (B [N, K]) or C = A B (B [K, N])

_CANDIDATES = {}  # (device index, op, N, K) -> [solution, ...]
_CHOICE = {}      # (device index, op, N, K, bucket) -> solution


def _bucket(M):
    return -(-M // BUCKET)


def _dims(a, b, op):
    M, K = a.shape
    if op == NT:
        N, Kb = b.shape
    else:
        Kb, N = b.shape
    if Kb != K:
        raise ValueError(f"inner dimensions differ: {K} vs {Kb}")
    return M, N, K


def _check(t, name, dev):
    _need(t, name, torch.float16, dev, contiguous=False)
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D fp16 tensor with unit column stride")
    return t.stride(0)


def choice(dev_index, op, N, K, M):
    """The solution used for this problem: the tuned one for M's bucket, else the nearest tuned
    bucket's, else torch's matmul."""
    b = _bucket(M)
    sol = _CHOICE.get((dev_index, op, N, K, b))
    if sol is not None:
        return sol
    near = [k[4] for k in _CHOICE if k[:4] == (dev_index, op, N, K)]
    if not near:
        return TORCH
    nb = min(near, key=lambda x: (abs(x - b), x))
    return _CHOICE[(dev_index, op, N, K, nb)]


def _run(sol, op, a, b, out, alpha, beta, M, N, K, lda, ldb, ldc, dev):
    _lib.call("qlora_gemm", op, M, N, K, _ptr(a), lda, _ptr(b), ldb, _ptr(out), ldc,
              float(alpha), float(beta), int(sol), _stream(dev))


def mm(a, b, op, out=None, bias=None):
    """fp16 [M, N] = a b^T (op NT, b [N, K]) or a b (op NN, b [K, N]) [+ bias, one rounding];
    a, b, out with unit column stride."""
    dev = a.device
    lda = _check(a, "a", dev)
    ldb = _check(b, "b", dev)
    M, N, K = _dims(a, b, op)
    if out is None:
        out = torch.empty((M, N), device=dev, dtype=torch.float16)
    ldc = _check(out, "out", dev)
    if out.shape != (M, N):
        raise ValueError(f"out must be [{M}, {N}]")
    if bias is not None:
        _need(bias, "bias", torch.float16, dev)
        if bias.numel() != N:
            raise ValueError("bias must have one entry per output column")
    if M == 0:
        return out
    sol = choice(dev.index or 0, op, N, K, M)
    if sol == TORCH:
        bt = b.t() if op == NT else b
        if bias is not None:
            return torch.addmm(bias, a, bt, out=out)
        return torch.mm(a, bt, out=out)
    beta = 0.0
    if bias is not None:
        out.copy_(bias.view(1, N).expand(M, N))
        beta = 1.0
    try:
        _run(sol, op, a, b, out, 1.0, beta, M, N, K, lda, ldb, ldc, dev)
    except RuntimeError:
        if sol == DEFAULT:
            raise
        # the bucket's solution rejects this exact size (rocBLAS checks before launching)
        _CHOICE[(dev.index or 0, op, N, K, _bucket(M))] = DEFAULT
        _run(DEFAULT, op, a, b, out, 1.0, beta, M, N, K, lda, ldb, ldc, dev)
    return out


def solutions(op, a, b, out):
    """Every rocBLAS solution index for this problem."""
    dev = a.device
    lda, ldb, ldc = _check(a, "a", dev), _check(b, "b", dev), _check(out, "out", dev)
    M, N, K = _dims(a, b, op)
    cnt = ctypes.c_int32(0)
    _lib.call("qlora_gemm_solutions", op, M, N, K, _ptr(a), lda, _ptr(b), ldb, _ptr(out), ldc,
              None, 0, ctypes.byref(cnt))
    if cnt.value == 0:
        return []
    arr = (ctypes.c_int32 * cnt.value)()
    _lib.call("qlora_gemm_solutions", op, M, N, K, _ptr(a), lda, _ptr(b), ldb, _ptr(out), ldc,
              arr, cnt.value, ctypes.byref(cnt))
    return list(arr)[:cnt.value]


def _time(fn, reps):
    fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps


def tune(shapes, Ms, device, top=6, reps=3, log=None):
    """Measure, for each (op, N, K) in shapes and each token count in Ms, the fastest of: torch's
    matmul, rocBLAS's default, and the `top` solutions that were fastest at the median token
    count. Buckets already tuned are skipped. Returns the seconds spent."""
    t0 = time.perf_counter()
    dev = torch.device(device)
    di = dev.index or 0
    buckets = sorted({_bucket(M) for M in Ms if M > 0})
    if not buckets:
        return 0.0
    work = [(op, N, K, [bk for bk in buckets if (di, op, N, K, bk) not in _CHOICE])
            for op, N, K in shapes]
    work = [w for w in work if w[3]]
    if not work:
        return 0.0
    m_max = buckets[-1] * BUCKET
    g = torch.Generator(device=dev).manual_seed(0)
    for op, N, K, todo in work:
        a_full = torch.randn((m_max, K), device=dev, generator=g).to(torch.float16)
        bshape = (N, K) if op == NT else (K, N)
        b = (torch.randn(bshape, device=dev, generator=g) * 0.02).to(torch.float16)
        c_full = torch.empty((m_max, N), device=dev, dtype=torch.float16)
        ldb = b.stride(0)

        def runner(sol, M):
            a, c = a_full[:M], c_full[:M]
            if sol == TORCH:
                bt = b.t() if op == NT else b
                return lambda: torch.mm(a, bt, out=c)
            return lambda: _run(sol, op, a, b, c, 1.0, 0.0, M, N, K, K, ldb, N, dev)

        key = (di, op, N, K)
        if key not in _CANDIDATES:
            m_mid = todo[len(todo) // 2] * BUCKET
            timed = []
            for sol in solutions(op, a_full[:m_mid], b, c_full[:m_mid]):
                try:
                    timed.append((_time(runner(sol, m_mid), 1), sol))
                except RuntimeError:
                    continue  # a solution that rejects the problem is not a candidate
            timed.sort()
            _CANDIDATES[key] = [TORCH, DEFAULT] + [s for _, s in timed[:top] if s != DEFAULT]
        for bk in todo:
            M = bk * BUCKET
            valid = set(solutions(op, a_full[:M], b, c_full[:M])) | {TORCH, DEFAULT}
            best = min((_time(runner(sol, M), reps), sol) for sol in _CANDIDATES[key]
                       if sol in valid)
            _CHOICE[key + (bk,)] = best[1]
            if log is not None:
                log(f"gemm tune op={op} N={N} K={K} M={M}: solution {best[1]} "
                    f"{best[0] * 1e3:.1f} us")
        del a_full, b, c_full
    return time.perf_counter() - t0


def reset():
    """Forget every measurement (tests)."""
    _CANDIDATES.clear()
    _CHOICE.clear()
