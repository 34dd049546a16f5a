"""GPU tests of the model-level decode: DualModLM (models/dualmod/model.py:134-313) on the HIP
attention path and the one-graph-per-token GraphDecoder (lm/eval/graph_decode.py:15-125).

* the device-position decode step (dm_decode_args.pos_dev) equals the host-position step bit
  for bit, over multi-split tapes and with a local window;
* dm_argmax_rows equals torch.argmax (first index on ties); dm_residual_rmsnorm adds exactly
  and normalises as the oracle's RMSNorm;
* the eager LM decode and the LM forward match the oracle's fp64 model (fp32, 1e-5);
* the graph's replays equal the eager decode_step bit for bit (logits, next token, tapes), with
  eager steps between the replays, and greedy generation gives the same tokens;
* the bf16 graph decode against the oracle: the reference validator's criteria
  (lm/eval/validate_graph_decode.py:97) restated for random weights — relative logit error
  within the bf16 bound, and the same argmax wherever the oracle's top-1 margin exceeds
  twice the measured logit error.
"""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.config import DualModConfig
from dual_mod_public_amd.decode import StaticTape
from dual_mod_public_amd.graph_decode import GraphDecoder
from dual_mod_public_amd.model import DualModLM
from dual_mod_public_amd.synthetic import make_lm_state_dict
from tests.hip_helpers import DEV, cfg_of, record, relerr, say, setup, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def _lm_cfg(**kw):
    base = dict(d_model=256, n_heads=4, n_layers=2, vocab_size=512, max_seq_len=64, mlp_hidden_override=512,
                checkpoint_chunk=0, dtype="fp32", ctx_mod="mult_res")
    base.update(kw)
    return DualModConfig(**base)


def _lm(cfg, dtype, seed=7):
    sd = make_lm_state_dict(cfg, seed=seed, std=0.02)
    m = DualModLM(cfg, dtype=dtype).to(DEV)
    m.load_state_dict({k: v.to(DEV) for k, v in sd.items()})
    return m.eval(), {k: v.double() for k, v in sd.items()}


def _tokens(cfg, B, T, seed=3):
    return torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(seed))


# the knob cases: linear and fusion write V rows from other epilogue branches; a k_ctx norm or the
# v'' clamp take the staged path (RoPE rows gathered, refined pair committed by its own kernel)
@pytest.mark.parametrize("dtype,P0,W,knobs", [
    (torch.float32, 0, 0, {}), (torch.bfloat16, 1500, 0, {}), (torch.bfloat16, 700, 300, {}),
    (torch.float32, 40, 8, {}), (torch.bfloat16, 600, 0, {"ctx_mod": "linear"}),
    (torch.bfloat16, 600, 0, {"ctx_mod": "fusion"}), (torch.bfloat16, 600, 0, {"k_ctx_norm": "rms"}),
    (torch.float32, 40, 0, {"v_clamp_tau": 0.5})])
def test_device_position_equals_host_position(dtype, P0, W, knobs):
    say(f"device-position decode vs host position dtype={dtype} P0={P0} W={W} {knobs}")
    cfg = cfg_of(d=256, h=4, T=P0 + 8, local_window=W, **knobs)
    B, steps = 3, 4
    P = P0 + steps
    sd, x, _, (c32, s32) = setup(cfg, B, P)
    g = torch.Generator().manual_seed(5)
    K0 = torch.randn(B, 4, P, 64, generator=g).to(dtype)
    V0 = torch.randn(B, 4, P, 64, generator=g).to(dtype)
    tapes = [StaticTape(cfg, B, P, DEV, dtype, sd=to_dev(sd, dtype)) for _ in range(2)]
    for t in tapes:
        t.K.copy_(K0.to(DEV))
        t.V.copy_(V0.to(DEV))
    pos_dev = torch.full((1,), P0, dtype=torch.int32, device=DEV)
    xd = x.to(DEV, dtype)
    for p in range(P0, P):
        o_h, y_h = tapes[0].step(xd[:, p].contiguous(), p, c32, s32, with_wo=True)
        o_h, y_h = o_h.clone(), y_h.clone()
        o_d, y_d = tapes[1].step(xd[:, p].contiguous(), pos_dev, c32, s32, with_wo=True)
        pos_dev += 1
        torch.cuda.synchronize()
        assert torch.equal(o_h, o_d) and torch.equal(y_h, y_d), p
    assert torch.equal(tapes[0].K, tapes[1].K) and torch.equal(tapes[0].V, tapes[1].V)


# aligned rows (the vector kernel, with and without a tail of columns) and an odd row stride (the
# scalar scan)
@pytest.mark.parametrize("cols,ld", [(32000, 32000), (31997, 32000), (31997, 31997)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_rows_matches_torch(dtype, cols, ld):
    say(f"dm_argmax_rows {dtype} cols={cols} ld={ld}")
    g = torch.Generator().manual_seed(1)
    x = torch.randn(37, ld, generator=g).to(dtype)
    x[3, 100] = x[3, cols - 1] = 50.0     # ties: the first index wins
    x[4, :] = 0.0
    x[5, 0] = 9.0
    x[6, cols - 1] = 60.0                 # the maximum in the last column (a tail column when cols % 8)
    x[7, cols:] = 99.0                    # past cols: not part of the row
    x[8, 17] = x[8, 40] = float("nan")    # a NaN is the maximum, the first NaN wins (torch.argmax)
    x[8, 5] = 80.0
    x[9, :] = float("-inf")               # all -inf: index 0
    x[10, cols - 2] = float("nan")        # a NaN in a late column beats a larger value earlier
    x[10, 3] = 70.0
    xd = x.to(DEV)
    out = torch.empty(37, dtype=torch.long, device=DEV)
    L.check(L.lib().dm_argmax_rows(L.dtype_code(dtype), L.ptr(xd), 37, cols, ld, L.ptr(out), L.stream_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), x[:, :cols].float().argmax(-1))
    assert out[3].item() == 100 and out[4].item() == 0 and out[5].item() == 0 and out[6].item() == cols - 1
    assert out[8].item() == 17 and out[9].item() == 0 and out[10].item() == cols - 2


# row lengths for the register-resident kernel (up to 4096: 4 and 16 values per thread) and the
# streaming one (longer rows)
@pytest.mark.parametrize("d", [1000, 3000, 5000])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_residual_rmsnorm(dtype, d):
    """dm_residual_rmsnorm: the residual add is exact fp32 (x + delta), the norm matches the
    oracle's RMSNorm (attention.py:74-83) in fp64 up to the output dtype's rounding."""
    say(f"dm_residual_rmsnorm {dtype} d={d}")
    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 1, d, generator=g) * 3
    delta = torch.randn(5, 1, d, generator=g).to(dtype)
    w = torch.rand(d, generator=g) + 0.5
    xd = x.to(DEV)
    y = L.residual_rmsnorm(xd, delta.to(DEV), w.to(DEV), dtype)
    torch.cuda.synchronize()
    xs = x + delta.float()
    assert torch.equal(xd.cpu(), xs)
    ref = O.rms_norm(xs.double(), w.double(), 1e-5)
    tol = 1e-6 if dtype == torch.float32 else 8e-3
    assert relerr(y, ref) < tol
    assert L.residual_rmsnorm(xd, None, None, dtype) is None    # nothing to add, no norm: a no-op
    assert torch.equal(xd.cpu(), xs)


def test_lm_decode_and_forward_match_oracle_fp32():
    say("DualModLM fp32: decode_step and forward vs the oracle's fp64 model")
    cfg = _lm_cfg()
    m, sd = _lm(cfg, torch.float32)
    B, T = 2, 24
    idx = _tokens(cfg, B, T)
    c64, s64 = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=torch.float64)
    ref = O.lm_forward(cfg, sd, idx, c64, s64)
    caches = m.decode_init()
    with torch.no_grad():
        dec = torch.cat([m.decode_step(idx[:, t:t + 1].to(DEV), t, caches) for t in range(T)], 1)
        fwd, _ = m(idx.to(DEV))
    torch.cuda.synchronize()
    e_dec, e_fwd = relerr(dec, ref), relerr(fwd, ref)
    record("lm_decode_forward_fp32", {"decode": e_dec, "forward": e_fwd}, 1e-5)
    say(f"  relerr decode {e_dec:.2e} forward {e_fwd:.2e}")
    assert e_dec < 1e-5 and e_fwd < 1e-5


# bf16 at B = 3 and 17 takes the MLP through dm_swiglu_rows (one and two row tiles), B = 65 (more
# rows than it takes) and fp32 through torch's products
@pytest.mark.parametrize("dtype,B", [(torch.float32, 3), (torch.bfloat16, 3), (torch.bfloat16, 17),
                                     (torch.bfloat16, 65)])
def test_graph_decoder_equals_eager(dtype, B):
    say(f"GraphDecoder replays vs eager decode_step, {dtype}, B={B}")
    cfg = _lm_cfg()
    m, _ = _lm(cfg, dtype)
    T = 40
    idx = _tokens(cfg, B, T, seed=4).to(DEV)
    dec = GraphDecoder(m, B, 48).capture()
    caches = m.decode_init()
    with torch.no_grad():
        for p in range(T):
            eag = m.decode_step(idx[:, p:p + 1], p, caches)        # eager work between the replays
            dec.tok.copy_(idx[:, p:p + 1])
            dec.step()
            torch.cuda.synchronize()
            assert torch.equal(dec.logits, eag.float()), p
            assert torch.equal(dec.next[:, 0].cpu(), eag.float().argmax(-1)[:, 0].cpu()), p
    assert int(dec.pos.item()) == T
    for l in range(cfg.n_layers):
        assert torch.equal(dec.K[l][:, :, :T], caches[l]["K"]) and torch.equal(dec.V[l][:, :, :T], caches[l]["V"])


def test_graph_decoder_follows_parameter_updates():
    """An in-place parameter update between replays (an optimizer step) is picked up by the next
    step: the graph's static weight copies are re-read when a parameter's version changes."""
    say("GraphDecoder after in-place parameter updates vs eager decode_step, bf16")
    cfg = _lm_cfg()
    m, _ = _lm(cfg, torch.bfloat16)
    B, T = 3, 12
    idx = _tokens(cfg, B, T, seed=8).to(DEV)
    dec = GraphDecoder(m, B, 16).capture()
    caches = m.decode_init()
    g = torch.Generator(device=DEV).manual_seed(9)
    with torch.no_grad():
        for p in range(T):
            if p in (3, 7):   # MLP, head (tied embedding) and attention weights all change
                for prm in (m.blocks[0].mlp.w2.weight, m.lm_head.weight, m.blocks[-1].attn.w_kctx.weight):
                    prm.add_(0.05 * torch.randn(prm.shape, generator=g, device=DEV))
            eag = m.decode_step(idx[:, p:p + 1], p, caches)
            dec.tok.copy_(idx[:, p:p + 1])
            dec.step()
            torch.cuda.synchronize()
            assert torch.equal(dec.logits, eag.float()), p


def test_graph_generate_equals_eager_greedy():
    say("GraphDecoder.generate vs eager greedy decode, bf16")
    cfg = _lm_cfg()
    m, _ = _lm(cfg, torch.bfloat16)
    B, Lp, n = 4, 12, 20
    prompt = _tokens(cfg, B, Lp, seed=6).to(DEV)
    dec = GraphDecoder(m, B, 40).capture()
    gen, k = dec.generate(prompt, n, check_every=8)
    assert k == n
    caches = m.decode_init()
    with torch.no_grad():
        for p in range(Lp):
            lg = m.decode_step(prompt[:, p:p + 1], p, caches)
        outs = []
        for j in range(n):
            nxt = lg[:, -1].float().argmax(-1, keepdim=True)
            outs.append(nxt)
            lg = m.decode_step(nxt, Lp + j, caches)
    assert torch.equal(gen, torch.cat(outs, 1).cpu())


def test_graph_decoder_bf16_vs_oracle():
    say("GraphDecoder bf16 teacher-forced vs the oracle's fp64 model")
    cfg = _lm_cfg()
    m, sd = _lm(cfg, torch.bfloat16)
    B, T = 4, 48
    idx = _tokens(cfg, B, T, seed=8)
    dec = GraphDecoder(m, B, 64).capture()
    outs = []
    for p in range(T):
        dec.tok.copy_(idx[:, p:p + 1].to(DEV))
        dec.step()
        outs.append(dec.logits.clone())
    got = torch.cat(outs, 1).double().cpu()
    c64, s64 = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=torch.float64)
    ref = O.lm_forward(cfg, sd, idx, c64, s64)
    err = relerr(got, ref)
    dmax = (got - ref).abs().max().item()
    top2 = ref.topk(2, -1).values
    margin = top2[..., 0] - top2[..., 1]
    decided = margin > 2 * dmax
    agree = (got.argmax(-1) == ref.argmax(-1))
    record("graph_decode_bf16", {"logits": err, "max_abs": dmax}, 2e-2)
    say(f"  relerr {err:.2e}  max|dlogit| {dmax:.4f}  argmax agree {agree.float().mean().item() * 100:.2f}% "
        f"({int(decided.sum())} of {decided.numel()} positions decided by more than 2 max|dlogit|)")
    assert err < 2e-2
    assert bool(agree[decided].all())


def test_graph_decoder_refuses_a_step_past_the_tape():
    say("GraphDecoder: a step past P_max is refused")
    cfg = _lm_cfg()
    m, _ = _lm(cfg, torch.bfloat16)
    dec = GraphDecoder(m, 2, 4).capture()
    for _ in range(4):
        dec.step()
    with pytest.raises(ValueError):
        dec.step()
    torch.cuda.synchronize()
    assert int(dec.pos.item()) == 4
    dec.reset()
    dec.step()
    torch.cuda.synchronize()
    assert int(dec.pos.item()) == 1


@pytest.mark.parametrize("M,d,H", [(1, 256, 512), (8, 1024, 2816), (16, 512, 1376), (5, 128, 96), (17, 256, 512),
                                   (40, 1024, 2816), (64, 512, 1376)])
def test_swiglu_rows_matches_fp32_reference(M, d, H):
    """dm_swiglu_rows (the decode step's MLP, models/dualmod/model.py:102-112) against the same
    products in fp32 on the bf16 inputs: act rounded once to bf16, so the bound is bf16's."""
    g = torch.Generator().manual_seed(M * 1000 + d + H)
    x = torch.randn(M, 1, d, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(H, d, generator=g) * d ** -0.5).to(torch.bfloat16)
    w3 = (torch.randn(H, d, generator=g) * d ** -0.5).to(torch.bfloat16)
    w2 = (torch.randn(d, H, generator=g) * H ** -0.5).to(torch.bfloat16)
    xf, w1f, w3f, w2f = (t.float() for t in (x, w1, w3, w2))
    ref = (torch.nn.functional.silu(xf @ w1f.T) * (xf @ w3f.T)) @ w2f.T
    act = torch.full((M, H), float("nan"), device=DEV, dtype=torch.bfloat16)
    out = L.swiglu_rows(x.to(DEV), w1.to(DEV), w3.to(DEV), w2.to(DEV), act=act)
    assert out.shape == x.shape and out.dtype == torch.bfloat16
    err = relerr(out.float().cpu(), ref)
    record(f"swiglu_rows M={M} d={d} H={H}", {"out": err}, 1e-2)
    assert err < 1e-2, err
    # deterministic: a second call gives the same bits
    out2 = L.swiglu_rows(x.to(DEV), w1.to(DEV), w3.to(DEV), w2.to(DEV))
    assert torch.equal(out, out2)
