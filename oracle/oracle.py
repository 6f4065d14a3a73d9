"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the reported CPU baseline.
The product package (vates_amd) never imports it.
"""
from __future__ import annotations

import ctypes
import math
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
IRWIN_HALL_STD = math.sqrt(4.0 * (65536.0 ** 2 - 1.0) / 12.0)

ORC_OK, ORC_EINVAL, ORC_ESLOT, ORC_ENOMEM = 0, -1, -2, -3

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.orc_f32_to_bf16.argtypes = [c_float]
        _lib.orc_bf16_to_f32.restype = c_float
        _lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _chk(rc, what):
    if rc != ORC_OK:
        raise RuntimeError(f"oracle {what} failed with {rc}")


def scale_for(std: float) -> float:
    return std / IRWIN_HALL_STD


def philox(ctr, key):
    c = (c_uint32 * 4)(*ctr)
    k = (c_uint32 * 2)(*key)
    o = (c_uint32 * 4)()
    lib().orc_philox4x32_10(c, k, o)
    return list(o)


def synth_normal(seed: int, stream: int, n: int, std: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_synth_normal(c_uint64(seed), c_uint32(stream), c_uint64(n), c_float(scale_for(std)), _p(out))
    return out


def synth_bf16(seed: int, stream: int, shape, std: float) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    lib().orc_synth_normal_bf16(c_uint64(seed), c_uint32(stream), c_uint64(n), c_float(scale_for(std)), _p(out))
    return out.reshape(shape)


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even, as orc_f32_to_bf16."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def quantize(w: np.ndarray, group: int = 64, bits: int = 4):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    wq = np.zeros((rows, cols * bits // 32), dtype=np.uint32)
    s = np.zeros((rows, cols // group), dtype=np.uint16)
    b = np.zeros_like(s)
    _chk(lib().orc_quantize_affine(_p(w), rows, cols, group, bits, _p(wq), _p(s), _p(b)), "quantize")
    return wq, s, b


def synth_quantized(seed: int, stream: int, rows: int, cols: int, group: int = 64, bits: int = 4, std: float = 0.02):
    wq = np.zeros((rows, cols * bits // 32), dtype=np.uint32)
    s = np.zeros((rows, cols // group), dtype=np.uint16)
    b = np.zeros_like(s)
    _chk(lib().orc_synth_quantized(c_uint64(seed), c_uint32(stream), rows, cols, group, bits,
                                   c_float(scale_for(std)), _p(wq), _p(s), _p(b)), "synth_quantized")
    return wq, s, b


def dequant(wq, s, b, rows, cols, group=64, bits=4) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    _chk(lib().orc_dequant_affine(_p(np.ascontiguousarray(wq, np.uint32)), _p(np.ascontiguousarray(s, np.uint16)),
                                  _p(np.ascontiguousarray(b, np.uint16)), rows, cols, group, bits, _p(out)), "dequant")
    return out


def qgemv_f64(wq, s, b, rows, cols, x, group=64, bits=4) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.empty((T, rows), dtype=np.float64)
    _chk(lib().orc_qgemv_f64(_p(wq), _p(s), _p(b), rows, cols, group, bits, _p(x), T, _p(y)), "qgemv")
    return y


def router_logits(wq, s, b, x_bf16, E, H, group=64, bits=8, bias=None) -> np.ndarray:
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    T = x_bf16.size // H
    out = np.empty((T, E), dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    _chk(lib().orc_router_logits_f32(_p(wq), _p(s), _p(b), _p(bias), E, H, group, bits, _p(x_bf16), T, _p(out)),
         "router")
    return out


def topk_softmax(logits, k, norm=True):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    ids = np.empty((T, k), dtype=np.int32)
    sc = np.empty((T, k), dtype=np.float32)
    _chk(lib().orc_topk_softmax(_p(logits), T, E, k, int(norm), _p(ids), _p(sc)), "topk")
    return ids, sc


def fused_moe_slots(x, slots, scores, pool, T, k, H, I, cap, group=64, bits=4):
    """pool: dict with gate_w/gate_s/gate_b/up_*/down_* numpy arrays."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    slots = np.ascontiguousarray(slots, dtype=np.int32)
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    out = np.empty((T, H), dtype=np.float32)
    rc = lib().orc_fused_moe_slots(_p(x), _p(slots), _p(scores), _p(pool["gate_w"]), _p(pool["gate_s"]),
                                   _p(pool["gate_b"]), _p(pool["up_w"]), _p(pool["up_s"]), _p(pool["up_b"]),
                                   _p(pool["down_w"]), _p(pool["down_s"]), _p(pool["down_b"]), T, k, H, I, group, bits,
                                   cap, _p(out))
    _chk(rc, "fused_moe_slots")
    return out


def moe_layer(x_bf16, L: dict, residual=False):
    """Full layer.  L holds numpy arrays and ints: H, I, E, k, group, norm,
    router_w/s/b, router_bits, bias (or None), table (or None), cap,
    gate_*/up_*/down_*, bits, and optionally sh_gate_*/sh_up_*/sh_down_*,
    sg_w/s/b, sg_bits, norm_w (bf16 bits or None), norm_eps.
    Returns (out_f32, out_bf16, ids, scores, slots)."""
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    H, k = L["H"], L["k"]
    T = x_bf16.size // H
    out_f32 = np.empty((T, H), dtype=np.float32)
    out_bf16 = np.empty((T, H), dtype=np.uint16)
    ids = np.empty((T, k), dtype=np.int32)
    sc = np.empty((T, k), dtype=np.float32)
    sl = np.empty((T, k), dtype=np.int32)
    g = L.get
    rc = lib().orc_moe_layer(
        _p(x_bf16), T, H, L["I"], L["E"], k, L["group"], int(L["norm"]),
        _p(L["router_w"]), _p(L["router_s"]), _p(L["router_b"]), L["router_bits"], _p(g("bias")), _p(g("table")),
        L["cap"], _p(L["gate_w"]), _p(L["gate_s"]), _p(L["gate_b"]), _p(L["up_w"]), _p(L["up_s"]), _p(L["up_b"]),
        _p(L["down_w"]), _p(L["down_s"]), _p(L["down_b"]), L["bits"],
        _p(g("sh_gate_w")), _p(g("sh_gate_s")), _p(g("sh_gate_b")), _p(g("sh_up_w")), _p(g("sh_up_s")),
        _p(g("sh_up_b")), _p(g("sh_down_w")), _p(g("sh_down_s")), _p(g("sh_down_b")),
        _p(g("sg_w")), _p(g("sg_s")), _p(g("sg_b")), g("sg_bits", 8), _p(g("norm_w")), c_float(g("norm_eps", 1e-6)),
        int(residual),
        _p(out_f32), _p(out_bf16), _p(ids), _p(sc), _p(sl))
    _chk(rc, "moe_layer")
    return out_f32, out_bf16, ids, sc, sl


def expert_major_groups(route_ids, num_experts, max_group_experts, max_assignments=32768):
    route_ids = np.ascontiguousarray(route_ids, dtype=np.int32).reshape(-1)
    counts = np.zeros(num_experts, dtype=np.int32)
    experts = np.zeros(num_experts, dtype=np.int32)
    nexp = np.zeros(1, dtype=np.int32)
    gstart = np.zeros(num_experts + 1, dtype=np.int32)
    gassign = np.zeros(num_experts + 1, dtype=np.int32)
    ng = lib().orc_expert_major_groups(_p(route_ids), route_ids.size, num_experts, max_group_experts, max_assignments,
                                       _p(counts), _p(experts), _p(nexp), _p(gstart), _p(gassign))
    if ng < 0:
        raise RuntimeError("expert_major_groups failed")
    ne = int(nexp[0])
    groups = []
    for gi in range(ng):
        end = gstart[gi + 1] if gi + 1 < ng else ne
        groups.append((tuple(int(e) for e in experts[gstart[gi]:end]), int(gassign[gi])))
    return counts, groups


def route_reduce(previous, weighted, assignment_pos, k, bf16_acc=False):
    out = np.array(previous, dtype=np.float32, copy=True)
    weighted = np.ascontiguousarray(weighted, dtype=np.float32)
    pos = np.ascontiguousarray(assignment_pos, dtype=np.int32)
    tokens, hidden = out.shape
    _chk(lib().orc_route_reduce(_p(out), _p(weighted), _p(pos), pos.size, tokens, hidden, k, int(bf16_acc)),
         "route_reduce")
    return out


def accept_greedy(drafts, preds, mode=0):
    drafts = np.ascontiguousarray(drafts, dtype=np.int32)
    preds = np.ascontiguousarray(preds, dtype=np.int32)
    K = drafts.size
    emitted = np.zeros(K + 1, dtype=np.int32)
    n = np.zeros(1, dtype=np.int32)
    m = np.zeros(1, dtype=np.int32)
    acc = np.zeros(1, dtype=np.int32)
    _chk(lib().orc_accept_greedy(_p(drafts), _p(preds), K, mode, _p(emitted), _p(n), _p(m), _p(acc)), "accept")
    return list(emitted[: n[0]]), int(m[0]), int(acc[0])


def argmax_rows(logits):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, V = logits.shape
    out = np.empty(rows, dtype=np.int32)
    _chk(lib().orc_argmax_rows(_p(logits), rows, V, _p(out)), "argmax")
    return out


def accept_tree(paths, preds):
    paths = np.ascontiguousarray(paths, dtype=np.int32)
    preds = np.ascontiguousarray(preds, dtype=np.int32)
    P, K = paths.shape
    best = np.zeros(1, dtype=np.int32)
    emitted = np.zeros(K + 1, dtype=np.int32)
    n = np.zeros(1, dtype=np.int32)
    m = np.zeros(1, dtype=np.int32)
    acc = np.zeros(1, dtype=np.int32)
    _chk(lib().orc_accept_tree(_p(paths), _p(preds), P, K, _p(best), _p(emitted), _p(n), _p(m), _p(acc)), "tree")
    return int(best[0]), list(emitted[: n[0]]), int(m[0]), int(acc[0])


def rmsnorm_bf16(x_bf16, w_bf16, eps):
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    T, H = x_bf16.shape
    out = np.empty_like(x_bf16)
    inv = np.empty(T, dtype=np.float32)
    _chk(lib().orc_rmsnorm_bf16(_p(x_bf16), _p(np.ascontiguousarray(w_bf16, np.uint16)), c_float(eps), T, H,
                                _p(out), _p(inv)), "rmsnorm")
    return out, inv


def lm_head(x: np.ndarray, norm_w, eps: float, W: np.ndarray):
    """logits (float64 [T, V]) and |x||w| sums of rmsnorm(x) . W^T; x, norm_w, W
    are bf16 bit patterns (uint16)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    T, H = x.shape
    V = W.shape[0]
    nw = None if norm_w is None else np.ascontiguousarray(norm_w, dtype=np.uint16)
    logits = np.empty((T, V), dtype=np.float64)
    absdot = np.empty((T, V), dtype=np.float64)
    fn = lib().orc_lm_head_f64
    fn.argtypes = [c_void_p, c_int, c_int, c_void_p, c_float, c_void_p, c_int, c_void_p, c_void_p]
    _chk(fn(_p(x), T, H, _p(nw), c_float(eps), _p(W), V, _p(logits), _p(absdot)), "lm_head")
    return logits, absdot



def gdn_layer(x, G: dict, conv_in=None, state_in=None):
    """Gated DeltaNet block in float64: (out [T, H], conv rows [T, conv_dim],
    states [T, n_v, dv, dk]).  G: H, n_k, n_v, dk, dv, eps, bits, in_norm,
    qkvz_w/_s/_b, ba_w/_s/_b, out_w/_s/_b, conv_w (bf16 bits [conv_dim, 4]),
    A_log, dt_bias (float32 [n_v]), norm_w (bf16 bits [dv]); conv_in float64
    [3, conv_dim] (oldest first) or None; state_in float64 [n_v, dv, dk] or None."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    H, nk, nv, dk, dv = G["H"], G["n_k"], G["n_v"], G["dk"], G["dv"]
    T = x.size // H
    cd = 2 * nk * dk + nv * dv
    out = np.empty((T, H), dtype=np.float64)
    rows = np.empty((T, cd), dtype=np.float64)
    states = np.empty((T, nv, dv, dk), dtype=np.float64)
    ci = None if conv_in is None else np.ascontiguousarray(conv_in, dtype=np.float64)
    si = None if state_in is None else np.ascontiguousarray(state_in, dtype=np.float64)
    a = {k: (np.ascontiguousarray(v) if isinstance(v, np.ndarray) else v) for k, v in G.items()}
    fn = lib().orc_gdn_layer_f64
    fn.argtypes = [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_float] + [c_void_p] * 10 + \
        [c_int] + [c_void_p] * 9
    _chk(fn(_p(x), T, H, nk, nv, dk, dv, c_float(G["eps"]), _p(a["in_norm"]),
            _p(a["qkvz_w"]), _p(a["qkvz_s"]), _p(a["qkvz_b"]), _p(a["ba_w"]), _p(a["ba_s"]), _p(a["ba_b"]),
            _p(a["out_w"]), _p(a["out_s"]), _p(a["out_b"]), G["bits"], _p(a["conv_w"]),
            _p(np.ascontiguousarray(G["A_log"], np.float32)), _p(np.ascontiguousarray(G["dt_bias"], np.float32)),
            _p(a["norm_w"]), _p(ci), _p(si), _p(out), _p(rows), _p(states)), "gdn_layer")
    return out, rows, states


def sd_masses(logits_row, temperature: float, top_p: float):
    """Integer masses W (uint32 [V]), nucleus threshold, Z_S and Z of one row."""
    l = np.ascontiguousarray(logits_row, dtype=np.float32)
    V = l.size
    W = np.empty(V, dtype=np.uint32)
    th = (c_uint32 * 1)()
    zs = (c_uint64 * 1)()
    z = (c_uint64 * 1)()
    fn = lib().orc_sd_masses
    fn.argtypes = [c_void_p, c_int, c_float, c_float, c_void_p, c_void_p, c_void_p, c_void_p]
    _chk(fn(_p(l), V, c_float(temperature), c_float(top_p), _p(W), th, zs, z), "sd_masses")
    return W, int(th[0]), int(zs[0]), int(z[0])


def sample_top_p(logits, temperature: float, top_p: float, seed: int, offset: int) -> np.ndarray:
    l = np.ascontiguousarray(logits, dtype=np.float32)
    rows, V = l.shape
    out = np.empty(rows, dtype=np.int32)
    fn = lib().orc_sample_top_p
    fn.argtypes = [c_void_p, c_int, c_int, c_float, c_float, c_uint64, c_uint64, c_void_p]
    _chk(fn(_p(l), rows, V, c_float(temperature), c_float(top_p), c_uint64(seed), c_uint64(offset), _p(out)),
         "sample_top_p")
    return out


def accept_stochastic(target, draft, drafts, temperature: float, top_p: float, seed: int, offset: int):
    """(emitted tokens, matched, accepted_len) of speculative sampling."""
    t = np.ascontiguousarray(target, dtype=np.float32)
    K = t.shape[0] - 1
    V = t.shape[1]
    d = None if draft is None else np.ascontiguousarray(draft, dtype=np.float32)
    dr = np.ascontiguousarray(drafts, dtype=np.int32)
    res = np.zeros(4 + K + 1, dtype=np.int32)
    fn = lib().orc_accept_stochastic
    fn.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_float, c_uint64, c_uint64, c_void_p]
    _chk(fn(_p(t), _p(d), _p(dr), K, V, c_float(temperature), c_float(top_p), c_uint64(seed), c_uint64(offset),
            _p(res)), "accept_stochastic")
    n = int(res[0])
    return [int(v) for v in res[4:4 + n]], int(res[1]), int(res[2]), res


def moe_layer_routed(x_bf16, L: dict, ids, scores, residual=False):
    """orc_moe_layer with the routing given: (out_f32, out_bf16)."""
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    H, k = L["H"], L["k"]
    T = x_bf16.size // H
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(T, k)
    scores = np.ascontiguousarray(scores, dtype=np.float32).reshape(T, k)
    out_f32 = np.empty((T, H), dtype=np.float32)
    out_bf16 = np.empty((T, H), dtype=np.uint16)
    g = L.get
    rc = lib().orc_moe_layer_routed(
        _p(x_bf16), T, H, L["I"], L["E"], k, L["group"], _p(g("table")), L["cap"],
        _p(L["gate_w"]), _p(L["gate_s"]), _p(L["gate_b"]), _p(L["up_w"]), _p(L["up_s"]), _p(L["up_b"]),
        _p(L["down_w"]), _p(L["down_s"]), _p(L["down_b"]), L["bits"],
        _p(g("sh_gate_w")), _p(g("sh_gate_s")), _p(g("sh_gate_b")), _p(g("sh_up_w")), _p(g("sh_up_s")),
        _p(g("sh_up_b")), _p(g("sh_down_w")), _p(g("sh_down_s")), _p(g("sh_down_b")),
        _p(g("sg_w")), _p(g("sg_s")), _p(g("sg_b")), g("sg_bits", 8), _p(g("norm_w")), c_float(g("norm_eps", 1e-6)),
        int(residual), _p(ids), _p(scores), _p(out_f32), _p(out_bf16))
    _chk(rc, "moe_layer_routed")
    return out_f32, out_bf16


def attention_layer(x, A: dict, pos0: int, k_cache, v_cache):
    """Full-attention block in float64: (out [T, H], k_new [T, n_kv, 256], v_new).
    A: H, n_heads, n_kv, rope_dim, theta, eps, bits, in_norm, q/k/v/o _w/_s/_b,
    q_norm, k_norm (bf16 bits / packed arrays); caches bf16 bits [n_kv, max_len, 256]."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    H = A["H"]
    T = x.size // H
    n_kv = A["n_kv"]
    kc = np.ascontiguousarray(k_cache, dtype=np.uint16)
    vc = np.ascontiguousarray(v_cache, dtype=np.uint16)
    max_len = kc.shape[1]
    out = np.empty((T, H), dtype=np.float64)
    kn = np.empty((T, n_kv, 256), dtype=np.float64)
    vn = np.empty((T, n_kv, 256), dtype=np.float64)
    fn = lib().orc_attention_layer_f64
    fn.argtypes = [c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_float, c_void_p] + [c_void_p] * 12 + \
        [c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p]
    a = {k: (np.ascontiguousarray(v) if isinstance(v, np.ndarray) else v) for k, v in A.items()}
    _chk(fn(_p(x), T, H, A["n_heads"], n_kv, A["rope_dim"], c_float(A["theta"]), c_float(A["eps"]), _p(a["in_norm"]),
            _p(a["q_w"]), _p(a["q_s"]), _p(a["q_b"]), _p(a["k_w"]), _p(a["k_s"]), _p(a["k_b"]),
            _p(a["v_w"]), _p(a["v_s"]), _p(a["v_b"]), _p(a["o_w"]), _p(a["o_s"]), _p(a["o_b"]), A["bits"],
            _p(a["q_norm"]), _p(a["k_norm"]), pos0, _p(kc), _p(vc), max_len, _p(out), _p(kn), _p(vn)),
         "attention_layer")
    return out, kn, vn


def set_threads(n: int) -> int:
    """Threads of the oracle's OpenMP loops; returns the previous setting."""
    fn = lib().orc_set_threads
    fn.argtypes = [c_int]
    fn.restype = c_int
    return fn(int(n))

