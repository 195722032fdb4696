"""A Llama model written to a GGUF v3 file, read by qk_gguf_open, uploaded
(qk_gguf_upload, GGUF::upload of inferencer.cu:322-339) and wired by
qk_gguf_llama (FastRunner's lookups, inferencer.cu:1196-1214): the decode
drivers built from the file must give bit-identical logits to the same
weights passed directly, and the oracle's greedy tokens.  Norm gains are
random so a swapped attn_norm / ffn_norm / output_norm would show."""
import numpy as np
import pytest

import gguf_writer as gw
from conftest import rel_l2

pytestmark = pytest.mark.gpu

CFG = dict(dim=512, layers=2, heads=8, kv_heads=2, hidden=1024, vocab=1000, context=64, eps=1e-5,
           rope_theta=10000.0)


def _weights(workloads, synth, seed, untied):
    W = workloads.llama_weights(CFG, seed)
    dim = CFG["dim"]
    for l, L in enumerate(W["layers"]):
        L["attn_norm"] = 1.0 + 0.2 * synth.normal_f32(dim, seed, 500 + 2 * l)
        L["ffn_norm"] = 1.0 + 0.2 * synth.normal_f32(dim, seed, 501 + 2 * l)
    W["output_norm"] = 1.0 + 0.2 * synth.normal_f32(dim, seed, 499)
    if untied:
        W["output"] = synth.quant_matrix(12, dim, CFG["vocab"], seed, 498, 0.02)
        W["output_type"] = 12
    return W


@pytest.mark.parametrize("untied,alignment,int8", [(False, None, False), (True, 64, False), (True, 64, True)])
def test_runner_from_gguf_matches_direct_and_oracle(qk, torch_gpu, oracle, workloads, synth, tmp_path, untied,
                                                    alignment, int8):
    """With int8 (both INT8 switches, an untied Q4_K output matrix): each
    greedy step's embedding row comes from the final pick, decoded from the
    Q6_K token table while the head read the other matrix.  The INT8 logits
    bound is the INT8 decode tests' per-step one (an activation code that
    rounds the other way from the oracle's moves the logits ~1e-2)."""
    t = torch_gpu
    W = _weights(workloads, synth, 21, untied)
    path = tmp_path / "model.gguf"
    gw.llama_writer(CFG, W, workloads.tensor_shape, alignment=alignment,
                    tokens=[f"tok{i}" for i in range(CFG["vocab"])]).write(path)
    g = qk.GGUF(path)
    g.upload()
    # The device copy holds the file's bytes.
    emb = g.tensor("token_embd.weight")
    dev = qk.copy_to_host(emb.device, emb.bytes, np.uint8)
    assert dev.tobytes() == W["token_embd"].tobytes()
    assert emb.device % 16 == 0
    rf = qk.Runner.from_gguf(g, CFG["context"])
    assert rf.cfg == {k: (np.float32(v).item() if isinstance(v, float) else v) for k, v in CFG.items()}
    rd = qk.Runner(CFG, W)
    om = oracle.Llama(CFG, W)
    if int8:
        for r in (rf, rd, om):
            r.set_int8(True, True)
    kc, vc = workloads.llama_kv_prefill(CFG, 21, 6)
    rf.load_kv(kc, vc)
    rd.load_kv(kc, vc)
    om.load_cache(kc, vc, 6)
    tok = 7
    for pos in range(6, 18):
        a = rf.forward(tok, pos, True)
        b = rd.forward(tok, pos, True)
        o, lg = om.forward(tok, pos, True)
        la, lb = rf.logits(), rd.logits()
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos
        assert a == b == o, (pos, a, b, o)
        assert rel_l2(la, lg) < (5e-2 if int8 else 1e-4)
        tok = o
    rf.close()
    rd.close()
    g.close()


def test_batch_runner_from_gguf(qk, torch_gpu, workloads, synth, tmp_path):
    W = _weights(workloads, synth, 22, False)
    path = tmp_path / "model.gguf"
    gw.llama_writer(CFG, W, workloads.tensor_shape).write(path)
    g = qk.GGUF(path)
    g.upload()
    rows = 3 * CFG["context"]
    bf = qk.BatchRunner.from_gguf(g, CFG["context"], 4, rows)
    bd = qk.BatchRunner(CFG, W, 4, rows)
    tokens, pos, kv_row = [5, 900, 33], [0, 0, 0], [0, 64, 128]
    for step in range(4):
        a = bf.forward(tokens, pos, kv_row)
        b = bd.forward(tokens, pos, kv_row)
        assert a == b
        assert np.array_equal(bf.logits(3).view(np.uint32), bd.logits(3).view(np.uint32))
        tokens, pos = a, [p + 1 for p in pos]
    bf.close()
    bd.close()
    g.close()


def test_llama_lookup_rejects_wrong_tensors(qk, torch_gpu, workloads, synth, tmp_path):
    W = _weights(workloads, synth, 23, False)

    def status_of(edit):
        w = gw.llama_writer(CFG, W, workloads.tensor_shape)
        edit(w)
        path = tmp_path / "m.gguf"
        w.write(path)
        g = qk.GGUF(path)
        g.upload()
        try:
            g.llama(CFG["context"])
            return qk.QK_OK, ""
        except qk.QKError as e:
            return e.status, str(e)
        finally:
            g.close()

    def retype_norm(w):
        for t in w.tensors:
            if t["name"] == "blk.1.ffn_norm.weight":
                t["type"], t["dims"], t["data"] = 12, [256, 2], bytes(288)

    def reshape_k(w):
        for t in w.tensors:
            if t["name"] == "blk.0.attn_k.weight":
                t["dims"] = [t["dims"][0], t["dims"][1] // 2]
                t["data"] = t["data"][: len(t["data"]) // 2]

    def drop_down(w):
        w.tensors = [t for t in w.tensors if t["name"] != "blk.1.ffn_down.weight"]

    def drop_param(w):
        w.meta = [m for m in w.meta if b"llama.feed_forward_length" not in m]

    assert status_of(lambda w: None)[0] == qk.QK_OK
    st, msg = status_of(retype_norm)
    assert st == qk.QK_ERR_TYPE and "blk.1.ffn_norm.weight" in msg
    st, msg = status_of(reshape_k)
    assert st == qk.QK_ERR_SHAPE and "blk.0.attn_k.weight" in msg
    st, msg = status_of(drop_down)
    assert st == qk.QK_ERR_INVALID_ARG and "blk.1.ffn_down.weight" in msg
    st, msg = status_of(drop_param)
    assert st == qk.QK_ERR_INVALID_ARG and "feed_forward_length" in msg


def test_runner_from_gguf_int8_matches_direct(qk, torch_gpu, workloads, synth, tmp_path):
    """The reference's default INT8 modes on a model loaded from a GGUF file:
    bit-identical logits and tokens to the same weights passed directly."""
    W = _weights(workloads, synth, 24, False)
    path = tmp_path / "model.gguf"
    gw.llama_writer(CFG, W, workloads.tensor_shape).write(path)
    g = qk.GGUF(path)
    g.upload()
    rf = qk.Runner.from_gguf(g, CFG["context"])
    rd = qk.Runner(CFG, W)
    for r in (rf, rd):
        r.set_int8(True, True)
    kc, vc = workloads.llama_kv_prefill(CFG, 24, 4)
    rf.load_kv(kc, vc)
    rd.load_kv(kc, vc)
    tok = 11
    for pos in range(4, 12):
        a = rf.forward(tok, pos, True)
        b = rd.forward(tok, pos, True)
        assert a == b, pos
        assert np.array_equal(rf.logits().view(np.uint32), rd.logits().view(np.uint32)), pos
        tok = a
    rf.close()
    rd.close()
    g.close()
