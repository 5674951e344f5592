"""Residual stream kernels and the per-token decode graph on the GPU.

* qm_residual_rmsnorm / qm_residual_add against the oracle's
  qo_residual_rmsnorm (qwen38_add_in_place + qwen38_rms_norm(_rows),
  qwen38.metal:4250-4333): the fp32 residual add bit for bit, the bf16 norm
  within 1e-4 of max|ref| beyond the final rounding.
* qm_decode_layers (decode_layers, metal_runtime.rs:2022-2084) on a small
  model of DeltaNet and full-attention layers: bit-equal to the same token
  issued as separate entry-point calls, and every one of those calls, over
  three tokens, within 1e-4 of the oracle run on that call's own GPU inputs
  (beyond the final bf16 rounding for bf16 outputs; residual adds, history
  windows and appended Q8 rows bit for bit).
* qm_decode_graph: bit-equal to qm_decode_layers over five tokens (both
  history-parity variants), and QM_ERR_GRAPH_STALE once a captured buffer
  changes.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import assert_bf16_close, bf16_dev_to_f32, empty_bf16, from_dev, to_dev
from qm38 import (DecodeFullLayer, DecodeGraph, DecodeLinearLayer, DnConfig, QmError, RopeConfig, Runtime,
                  synth)

pytestmark = pytest.mark.gpu

EPS = 1e-6


# ---------------------------------------------------------------- RMSNorm --
@pytest.mark.parametrize("M,n", [(1, 5120), (3, 256), (2, 1002), (1, 6), (4, 64)])
@pytest.mark.parametrize("with_delta", [False, True])
def test_residual_rmsnorm_matches_oracle(rt, torch_dev, M, n, with_delta):
    rng = np.random.default_rng(M * 1000 + n + with_delta)
    h = (rng.standard_normal((M, n)) * 3).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    d_bits = synth.bf16_normal(rng, (M, n)) if with_delta else None
    hd = to_dev(h, torch_dev)
    out = empty_bf16((M, n), torch_dev)
    rt.residual_rmsnorm(hd, None if d_bits is None else to_dev(d_bits, torch_dev), to_dev(w, torch_dev), M, n,
                        EPS, out)
    h_ref, o_ref = oracle.residual_rmsnorm(h, w, EPS, None if d_bits is None else synth.bf16_to_f32(d_bits))
    np.testing.assert_array_equal(from_dev(hd), h_ref)
    assert_bf16_close(bf16_dev_to_f32(out), o_ref, what=f"rmsnorm M{M} n{n}")


def test_residual_add_exact(rt, torch_dev):
    rng = np.random.default_rng(5)
    h = rng.standard_normal(3000).astype(np.float32)
    d = synth.bf16_normal(rng, (3000,))
    hd = to_dev(h, torch_dev)
    rt.residual_add(hd, to_dev(d, torch_dev), 3000)
    np.testing.assert_array_equal(from_dev(hd), h + synth.bf16_to_f32(d))


def test_rmsnorm_rejects_bad_arguments(rt, torch_dev):
    import torch
    h = torch.zeros(64, dtype=torch.float32, device=torch_dev)
    w = torch.ones(64, dtype=torch.float32, device=torch_dev)
    o = torch.zeros(64, dtype=torch.int16, device=torch_dev)
    with pytest.raises(QmError, match="EMPTY"):
        rt.residual_rmsnorm(h, None, w, 0, 64, EPS, o)
    with pytest.raises(QmError):
        rt.residual_rmsnorm(h, None, None, 1, 64, EPS, o)
    with pytest.raises(QmError):
        rt.residual_rmsnorm(h, None, w, 1, 64, -1.0, o)


# ------------------------------------------------------------ toy model --
HID, INTER = 256, 512
DN = dict(key_heads=2, value_heads=4, key_head_dim=32, value_head_dim=32, conv_kernel_size=4)
FULL = dict(heads=4, kv_heads=2, head_dim=64, rotary_dim=16, theta=1e7)


def _q4(rng, rows, K):
    return synth.q4_matrix(rng, rows, K)


class Model:
    """Host copies of a small [linear, full, linear] model's weights plus their
    device uploads (shared by every state built from it)."""

    def __init__(self, rt, dev, seed=0, kinds=("linear", "full", "linear")):
        rng = np.random.default_rng(seed)
        self.kinds = kinds
        self.rt, self.dev = rt, dev
        c = DN
        self.channels = 2 * c["key_heads"] * c["key_head_dim"] + c["value_heads"] * c["value_head_dim"]
        self.value = c["value_heads"] * c["value_head_dim"]
        self.layers = []
        for kind in kinds:
            L = dict(kind=kind,
                     in_norm=(1 + 0.1 * rng.standard_normal(HID)).astype(np.float32),
                     post_norm=(1 + 0.1 * rng.standard_normal(HID)).astype(np.float32),
                     gate=_q4(rng, INTER, HID), up=_q4(rng, INTER, HID), down=_q4(rng, HID, INTER))
            if kind == "linear":
                L.update(qkv=_q4(rng, self.channels, HID), z=_q4(rng, self.value, HID),
                         b=_q4(rng, c["value_heads"], HID), a=_q4(rng, c["value_heads"], HID),
                         out=_q4(rng, HID, self.value),
                         conv=(0.3 * rng.standard_normal((self.channels, c["conv_kernel_size"]))).astype(np.float32),
                         a_log=(0.1 * rng.standard_normal(c["value_heads"])).astype(np.float32),
                         dt_bias=(0.1 * rng.standard_normal(c["value_heads"])).astype(np.float32),
                         norm=(1 + 0.1 * rng.standard_normal(c["value_head_dim"])).astype(np.float32))
            else:
                H, KVH, D = FULL["heads"], FULL["kv_heads"], FULL["head_dim"]
                L.update(q=_q4(rng, 2 * H * D, HID), k=_q4(rng, KVH * D, HID), v=_q4(rng, KVH * D, HID),
                         o=_q4(rng, HID, H * D),
                         q_norm=(1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
                         k_norm=(1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
            self.layers.append(L)
        self._dev = []  # device tensors kept alive
        self._alive = []  # states and caches of every request
        self.jobs = []
        self.dn_weights = []
        for L in self.layers:
            J = {}
            for key in ("gate", "up", "down", "qkv", "z", "b", "a", "out", "q", "k", "v", "o"):
                if key in L:
                    w, s, b = (to_dev(t, dev) for t in L[key])
                    self._dev += [w, s, b]
                    J[key] = Runtime.job(w, s, b, L[key][0].shape[0])
            for key in ("in_norm", "post_norm", "q_norm", "k_norm"):
                if key in L:
                    t = to_dev(L[key], dev)
                    self._dev.append(t)
                    J[key] = t
            self.jobs.append(J)
            if L["kind"] == "linear":
                cfg = DnConfig(c["key_heads"], c["value_heads"], c["key_head_dim"], c["value_head_dim"],
                               c["conv_kernel_size"])
                self.dn_weights.append(rt.create_deltanet_weights(cfg, L["conv"], L["a_log"], L["dt_bias"], L["norm"]))
            else:
                self.dn_weights.append(None)

    def rope(self):
        return RopeConfig(FULL["head_dim"], FULL["rotary_dim"], FULL["theta"], 2, 2, 1)  # M-RoPE sections (2, 2)

    def new_request(self, max_tokens=64):
        """Fresh DeltaNet states / KV caches and the layer descriptors over them."""
        states, caches, descs = [], [], []
        for L, J, W in zip(self.layers, self.jobs, self.dn_weights):
            if L["kind"] == "linear":
                st = W.create_state()
                states.append(st)
                caches.append(None)
                descs.append(DecodeLinearLayer(J["in_norm"].data_ptr(), J["post_norm"].data_ptr(), J["qkv"], J["z"],
                                               J["b"], J["a"], J["out"], W.handle.value, st.handle.value, J["gate"],
                                               J["up"],
                                               J["down"]))
            else:
                kv = self.rt.create_q8_kv_state(FULL["kv_heads"], FULL["head_dim"], max_tokens)
                states.append(None)
                caches.append(kv)
                descs.append(DecodeFullLayer(J["in_norm"].data_ptr(), J["post_norm"].data_ptr(), J["q"], J["k"],
                                             J["v"], J["o"], J["q_norm"].data_ptr(), J["k_norm"].data_ptr(),
                                             FULL["heads"], self.rope(), kv.handle.value, J["gate"], J["up"],
                                             J["down"]))
        # The descriptors hold raw handles: keep the objects alive with the model.
        self._alive.append((states, caches))
        return states, caches, descs


def _hidden0(seed):
    return (np.random.default_rng(seed).standard_normal(HID) * 2).astype(np.float32)


def _state_with(rt, dev, h):
    st = rt.create_decode_state(HID)
    rt.lib.qm_copy_to_device(rt.handle, st.hidden_ptr, h.ctypes.data, h.nbytes)
    return st


def _hidden(rt, st):
    out = np.zeros(HID, np.float32)
    rt.synchronize()
    rt.lib.qm_copy_to_host(rt.handle, out.ctypes.data, st.hidden_ptr, out.nbytes)
    return out


def _positions(t):
    return (t, t + 3, t + 7)  # distinct M-RoPE axes


def _manual_token(rt, dev, model, states, caches, hidden, pos):
    """The same token as separate entry-point calls (torch for the exact
    bf16 <-> fp32 conversions)."""
    import torch
    bf = lambda n: torch.empty(n, dtype=torch.int16, device=dev)  # noqa: E731

    def f32(t):
        return (t.to(torch.int32) & 0xFFFF).bitwise_left_shift(16).view(torch.float32)

    def to_bf(t):
        return t.to(torch.bfloat16).view(torch.int16)

    x = bf(HID)
    delta2 = None
    posd = torch.tensor(np.array(pos, np.uint32).view(np.int32), device=dev)
    for i, (L, J) in enumerate(zip(model.layers, model.jobs)):
        rt.residual_rmsnorm(hidden, delta2, J["in_norm"], 1, HID, EPS, x)
        delta = bf(HID)
        if L["kind"] == "linear":
            outs = [bf(model.channels), bf(model.value), bf(DN["value_heads"]), bf(DN["value_heads"])]
            rt.q4_project([J["qkv"], J["z"], J["b"], J["a"]], x, HID, 1, outs)
            dn_out = torch.empty(model.value, dtype=torch.float32, device=dev)
            rt.deltanet_step(model.dn_weights[i], states[i], *(f32(o) for o in outs), EPS, dn_out)
            rt.q4_project([J["out"]], to_bf(dn_out), model.value, 1, [delta])
        else:
            H, KVH, D = FULL["heads"], FULL["kv_heads"], FULL["head_dim"]
            qg, kb, vb = bf(2 * H * D), bf(KVH * D), bf(KVH * D)
            rt.q4_project([J["q"], J["k"], J["v"]], x, HID, 1, [qg, kb, vb])
            q, g = bf(H * D), bf(H * D)
            k = torch.empty(KVH * D, dtype=torch.float32, device=dev)
            rt.attn_prepare(model.rope(), 1, H, KVH, qg, kb, J["q_norm"], J["k_norm"], EPS, q, g, k, positions=posd)
            att = bf(H * D)
            rt.gqa_attention_q8([caches[i]], q, g, k, f32(vb), H, att)
            rt.q4_project([J["o"]], att, H * D, 1, [delta])
        rt.residual_rmsnorm(hidden, delta, J["post_norm"], 1, HID, EPS, x)
        h = bf(INTER)
        rt.q4_swiglu(J["gate"], J["up"], x, HID, 1, h)
        delta2 = bf(HID)
        rt.q4_project([J["down"]], h, INTER, 1, [delta2])
    rt.residual_add(hidden, delta2, HID)


def test_decode_layers_match_separate_calls(rt, torch_dev):
    import torch
    model = Model(rt, torch_dev, seed=11)
    h0 = _hidden0(1)
    states_a, caches_a, descs = model.new_request()
    st = _state_with(rt, torch_dev, h0)
    states_b, caches_b, _ = model.new_request()
    hidden_b = torch.from_numpy(h0.copy()).to(torch_dev)
    for t in range(3):
        rt.decode_layers(st, descs, _positions(t), EPS)
        _manual_token(rt, torch_dev, model, states_b, caches_b, hidden_b, _positions(t))
        np.testing.assert_array_equal(_hidden(rt, st), from_dev(hidden_b), err_msg=f"token {t}")
    for sa, sb in zip(states_a, states_b):
        if sa is not None:
            for x, y in zip(sa.read(), sb.read()):
                np.testing.assert_array_equal(x, y)
    for ca, cb in zip(caches_a, caches_b):
        if ca is not None:
            assert ca.sequence_length == cb.sequence_length == 3
            for x, y in zip(ca.read(), cb.read()):
                np.testing.assert_array_equal(x, y)


class _StageCheck:
    """Compares every kernel of a token with the oracle fed that kernel's own
    GPU inputs (the bf16 / fp32 intermediates the previous kernel stored), so
    each stage is held to its own bar instead of an end-to-end bound that
    has to absorb bf16 rounding-boundary flips carried through the layers:
    bf16 outputs within 1e-4 of max|ref| beyond their final rounding
    (assert_bf16_close), fp32 outputs within 1e-4 of max|ref|, residual adds
    and history windows bit for bit."""

    def __init__(self):
        self.stages = 0

    def bits(self, t):
        return from_dev(t, np.uint16).reshape(-1)

    def f32(self, t):
        return from_dev(t).reshape(-1).astype(np.float32)

    def bf16(self, t, ref, what):
        assert_bf16_close(bf16_dev_to_f32(t).reshape(-1), np.asarray(ref, np.float64).reshape(-1), what=what)
        self.stages += 1

    def close(self, got, ref, what, tol=1e-4):
        got = np.asarray(got, np.float64).reshape(-1)
        ref = np.asarray(ref, np.float64).reshape(-1)
        err = np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30)
        assert err <= tol, f"{what}: rel err {err:.3e} > {tol:.1e}"
        self.stages += 1

    def project(self, L, key, x_bits, out, what):
        self.bf16(out, oracle.q4_project(x_bits, *L[key])[0], f"{what} {key}")


def _checked_token(rt, dev, model, states, caches, hidden, pos, chk):
    """_manual_token's calls, each followed by its oracle check on the GPU's
    own inputs."""
    import torch
    bf = lambda n: torch.empty(n, dtype=torch.int16, device=dev)  # noqa: E731

    def f32(t):
        return (t.to(torch.int32) & 0xFFFF).bitwise_left_shift(16).view(torch.float32)

    def to_bf(t):
        return t.to(torch.bfloat16).view(torch.int16)

    def norm(delta, w, x, what):
        h_in = from_dev(hidden).copy()
        d_in = None if delta is None else synth.bf16_to_f32(chk.bits(delta))
        rt.residual_rmsnorm(hidden, delta, w, 1, HID, EPS, x)
        h_ref, x_ref = oracle.residual_rmsnorm(h_in, from_dev(w), EPS, d_in)
        np.testing.assert_array_equal(from_dev(hidden), h_ref[0], err_msg=f"{what} residual")
        chk.bf16(x, x_ref[0], f"{what} rmsnorm")

    x = bf(HID)
    delta2 = None
    H, KVH, D = FULL["heads"], FULL["kv_heads"], FULL["head_dim"]
    posd = torch.tensor(np.array(pos, np.uint32).view(np.int32), device=dev)
    for i, (L, J) in enumerate(zip(model.layers, model.jobs)):
        what = f"layer {i} ({L['kind']}) pos {pos[0]}"
        norm(delta2, J["in_norm"], x, what)
        xb = chk.bits(x)
        delta = bf(HID)
        if L["kind"] == "linear":
            keys = ("qkv", "z", "b", "a")
            outs = [bf(model.channels), bf(model.value), bf(DN["value_heads"]), bf(DN["value_heads"])]
            rt.q4_project([J[k] for k in keys], x, HID, 1, outs)
            for k, o in zip(keys, outs):
                chk.project(L, k, xb, o, what)
            hist, S = states[i].read()
            ins = [synth.bf16_to_f32(chk.bits(o))[None] for o in outs]
            dn_out = torch.empty(model.value, dtype=torch.float32, device=dev)
            rt.deltanet_step(model.dn_weights[i], states[i], *(f32(o) for o in outs), EPS, dn_out)
            ref, h_ref, S_ref = oracle.deltanet_prefill(DN, L["conv"], L["a_log"], L["dt_bias"], L["norm"], *ins, EPS,
                                                        hist, S, f64=True)
            chk.close(chk.f32(dn_out), ref[0], f"{what} deltanet out")
            h_got, S_got = states[i].read()
            np.testing.assert_array_equal(h_got, h_ref, err_msg=f"{what} conv history")
            chk.close(S_got, S_ref, f"{what} deltanet state")
            ob = to_bf(dn_out)
            rt.q4_project([J["out"]], ob, model.value, 1, [delta])
            chk.project(L, "out", chk.bits(ob), delta, what)
        else:
            qg, kb, vb = bf(2 * H * D), bf(KVH * D), bf(KVH * D)
            rt.q4_project([J["q"], J["k"], J["v"]], x, HID, 1, [qg, kb, vb])
            for k, o in zip(("q", "k", "v"), (qg, kb, vb)):
                chk.project(L, k, xb, o, what)
            q, g = bf(H * D), bf(H * D)
            k = torch.empty(KVH * D, dtype=torch.float32, device=dev)
            rt.attn_prepare(model.rope(), 1, H, KVH, qg, kb, J["q_norm"], J["k_norm"], EPS, q, g, k, positions=posd)
            rq, _, rk = oracle.attn_prepare(synth.bf16_to_f32(chk.bits(qg)).reshape(1, H, 2 * D),
                                            synth.bf16_to_f32(chk.bits(kb)).reshape(1, KVH, D), L["q_norm"],
                                            L["k_norm"], D, FULL["rotary_dim"], FULL["theta"], EPS, sections=(2, 2),
                                            positions=np.array(pos, np.uint32).reshape(3, 1))
            chk.bf16(q, rq, f"{what} prepared query")
            chk.close(chk.f32(k), rk, f"{what} prepared key", tol=2e-5)
            att = bf(H * D)
            rt.gqa_attention_q8([caches[i]], q, g, k, f32(vb), H, att)
            kq, vq, ks, vs = caches[i].read()
            # The appended row is the Q8 quantisation of the GPU's own fp32 key
            # and bf16-valued value, bit for bit.
            for got_q, got_s, row in ((kq, ks, chk.f32(k)), (vq, vs, synth.bf16_to_f32(chk.bits(vb)))):
                rq8, rs8 = oracle.q8_quantize_rows(row.reshape(1, KVH, D))
                np.testing.assert_array_equal(got_q[-1:], rq8, err_msg=f"{what} appended Q8 row")
                np.testing.assert_array_equal(got_s[-1:], rs8, err_msg=f"{what} appended Q8 scales")
            ref = oracle.attention(synth.bf16_to_f32(chk.bits(q)).reshape(1, H, D),
                                   synth.bf16_to_f32(chk.bits(g)).reshape(1, H, D), kq, ks, vq, vs, kq.shape[0] - 1)
            chk.bf16(att, ref, f"{what} attention")
            rt.q4_project([J["o"]], att, H * D, 1, [delta])
            chk.project(L, "o", chk.bits(att), delta, what)
        norm(delta, J["post_norm"], x, f"{what} post")
        xb = chk.bits(x)
        h = bf(INTER)
        rt.q4_swiglu(J["gate"], J["up"], x, HID, 1, h)
        chk.bf16(h, oracle.swiglu(oracle.q4_project(xb, *L["gate"]), oracle.q4_project(xb, *L["up"]))[0],
                 f"{what} swiglu")
        delta2 = bf(HID)
        rt.q4_project([J["down"]], h, INTER, 1, [delta2])
        chk.project(L, "down", chk.bits(h), delta2, what)
    h_in = from_dev(hidden).copy()
    rt.residual_add(hidden, delta2, HID)
    np.testing.assert_array_equal(from_dev(hidden), h_in + synth.bf16_to_f32(chk.bits(delta2)))


def test_decode_layers_match_oracle_stagewise(rt, torch_dev):
    """qm_decode_layers over three tokens, bit-equal each token to the same
    calls issued one by one, and each of those calls within its own bar of
    the oracle run on the GPU's inputs to it."""
    import torch
    model = Model(rt, torch_dev, seed=12)
    h0 = _hidden0(2)
    _, _, descs = model.new_request()
    st = _state_with(rt, torch_dev, h0)
    states_b, caches_b, _ = model.new_request()
    hidden_b = torch.from_numpy(h0.copy()).to(torch_dev)
    chk = _StageCheck()
    for t in range(3):
        rt.decode_layers(st, descs, _positions(t), EPS)
        _checked_token(rt, torch_dev, model, states_b, caches_b, hidden_b, _positions(t), chk)
        np.testing.assert_array_equal(_hidden(rt, st), from_dev(hidden_b), err_msg=f"token {t}")
    assert chk.stages == 3 * 3 * 11  # 11 stages in each of the three layers, three tokens


@pytest.mark.parametrize("kinds", [("linear", "full", "linear"), ("full", "full"), ("linear", "linear")])
def test_graph_matches_eager(rt, torch_dev, kinds):
    model = Model(rt, torch_dev, seed=13, kinds=kinds)
    h0 = _hidden0(3)
    states_a, caches_a, descs_a = model.new_request()
    states_b, caches_b, descs_b = model.new_request()
    st_a = _state_with(rt, torch_dev, h0)
    st_b = _state_with(rt, torch_dev, h0)
    g = DecodeGraph(rt, st_b, descs_b, EPS)
    for t in range(5):
        rt.decode_layers(st_a, descs_a, _positions(t), EPS)
        g.run(_positions(t))
        np.testing.assert_array_equal(_hidden(rt, st_b), _hidden(rt, st_a), err_msg=f"token {t}")
    for sa, sb in zip(states_a, states_b):
        if sa is not None:
            for x, y in zip(sa.read(), sb.read()):
                np.testing.assert_array_equal(x, y)
    for ca, cb in zip(caches_a, caches_b):
        if ca is not None:
            assert cb.sequence_length == 5
            for x, y in zip(ca.read(), cb.read()):
                np.testing.assert_array_equal(x, y)
    g.close()


def test_graph_stale_after_buffer_exchange(rt, torch_dev):
    model = Model(rt, torch_dev, seed=14, kinds=("linear", "full"))
    states, _, descs = model.new_request()
    st = _state_with(rt, torch_dev, _hidden0(4))
    g = DecodeGraph(rt, st, descs, EPS)
    g.run(_positions(0))
    # An eager token flips the history parity: the other variant still runs.
    rt.decode_layers(st, descs, _positions(1), EPS)
    g.run(_positions(2))
    # A one-row snapshot restore exchanges the state's buffers.
    snaps = model.dn_weights[0].create_snapshots(1)
    snaps.restore(0, states[0])
    with pytest.raises(QmError, match="changed after capture"):
        g.run(_positions(3))
    g.close()
    # Recapturing picks up the new buffers.
    g2 = DecodeGraph(rt, st, descs, EPS)
    g2.run(_positions(3))
    rt.synchronize()
    g2.close()


def test_decode_layers_reject_bad_layers(rt, torch_dev):
    model = Model(rt, torch_dev, seed=15, kinds=("linear", "full"))
    _, _, descs = model.new_request()
    st = _state_with(rt, torch_dev, _hidden0(5))
    bad = DecodeLinearLayer.from_buffer_copy(descs[0])
    bad.out_proj = bad.b  # wrong output rows
    with pytest.raises(QmError, match="WRONG_LENGTH|output rows"):
        rt.decode_layers(st, [bad, descs[1]], 0, EPS)
    badf = DecodeFullLayer.from_buffer_copy(descs[1])
    badf.num_heads = 3  # not a multiple of kv_heads
    with pytest.raises(QmError):
        rt.decode_layers(st, [descs[0], badf], 0, EPS)
    with pytest.raises(QmError):
        rt.decode_layers(st, [], 0, EPS)
    with pytest.raises(QmError):
        DecodeGraph(rt, st, [bad], EPS)


def test_graph_and_eager_report_kv_capacity(rt, torch_dev):
    # A (linear, full) model whose cache has a hard limit of two tokens: the
    # third token fails with CAPACITY_EXCEEDED, eagerly and from a graph
    # replay, before anything is launched, so the residual row, the DeltaNet
    # state (history, recurrence and history parity) and the cache are as
    # they were (decode_layers commits nothing on an encode error,
    # metal_runtime.rs:2022-2084).
    model = Model(rt, torch_dev, seed=16, kinds=("linear", "full"))
    states, caches, descs = model.new_request(max_tokens=2)
    st = _state_with(rt, torch_dev, _hidden0(6))
    rt.decode_layers(st, descs, _positions(0), EPS)
    g = DecodeGraph(rt, st, descs, EPS)
    g.run(_positions(1))
    rt.synchronize()
    assert caches[1].sequence_length == 2

    def snapshot():
        rt.synchronize()
        hist, rec = states[0].read()
        return _hidden(rt, st), hist.copy(), rec.copy(), caches[1].read()

    before = snapshot()
    with pytest.raises(QmError, match="CAPACITY|capacity"):
        g.run(_positions(2))
    with pytest.raises(QmError, match="CAPACITY|capacity"):
        rt.decode_layers(st, descs, _positions(2), EPS)
    after = snapshot()
    for x, y in zip(before[:3], after[:3]):
        np.testing.assert_array_equal(x, y)
    for x, y in zip(before[3], after[3]):
        np.testing.assert_array_equal(x, y)
    assert caches[1].sequence_length == 2
    # The history parity did not move: the graph's variant for it still runs
    # once the cache may grow again (a truncation makes room).
    caches[1].truncate(1)
    g.run(_positions(2))
    rt.synchronize()
    assert caches[1].sequence_length == 2
    g.close()
