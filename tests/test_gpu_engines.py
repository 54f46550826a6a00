"""ZeRO engines on the GPU (world_size 1).

- Optimizer arithmetic: with prescribed gradients, every stage's fp32 master
  after a step equals the oracle's EngineRef (zero/stage0_ddp.py:66-88 order)
  within 1e-5 relative, and the parameters equal the master rounded to bf16.
- Stage 3 behaviour the reference tests pin (zero/tests/test_zero_stages.py):
  resharding between calls, summon round trip, stage 3 == stage 0 training,
  checkpoint restore; stage 2 gradient release and memory accounting.
"""
from __future__ import annotations

import pytest
import torch

from collectives import LocalCollectives, TracingCollectives
from model import LlamaForCausalLM, ModelConfig
from oracle import engine as OE
from profiler import MemoryTracker
from zero import ZeROStage0DDP, ZeROStage1Optimizer, ZeROStage2Optimizer, ZeROStage3Optimizer
from lzhip import ops
from zero.common import assign_flat_params, build_flat_param_metadata, flatten_params_fp32

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
STAGES = {0: ZeROStage0DDP, 1: ZeROStage1Optimizer, 2: ZeROStage2Optimizer, 3: ZeROStage3Optimizer}


def _cfg(**kw) -> ModelConfig:
    base = dict(name="zero_test", vocab_size=97, max_seq_len=64, dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                ffn_dim=256, rope_theta=10_000.0)
    base.update(kw)
    return ModelConfig(**base)


def _batch(step: int, bsz: int = 3, seq: int = 64, vocab: int = 97) -> torch.Tensor:
    base = torch.arange(bsz * seq, dtype=torch.long).view(bsz, seq)
    return ((base * 7 + step * 13) % vocab).to(DEV)


def _model(seed: int, **kw) -> LlamaForCausalLM:
    torch.manual_seed(seed)
    return LlamaForCausalLM(_cfg(**kw)).to(device=DEV, dtype=torch.bfloat16)


def _full_params(engine, model):
    ctx = engine.summon_full_params() if hasattr(engine, "summon_full_params") else None
    if ctx is None:
        return {n: p.detach().float().clone() for n, p in model.named_parameters()}
    with ctx:
        return {n: p.detach().float().clone() for n, p in model.named_parameters()}


def test_assign_flat_params_reuses_storage():
    m = torch.nn.Sequential(torch.nn.Linear(4, 3), torch.nn.Linear(3, 2)).to(DEV)
    meta = build_flat_param_metadata(m)
    ptrs = [p.data.data_ptr() for p in meta.params]
    flat = flatten_params_fp32(meta)
    ref = torch.cat([p.detach().reshape(-1) for p in meta.params])
    assert torch.equal(flat, ref)
    assign_flat_params(meta, flat + 1.0)
    assert [p.data.data_ptr() for p in meta.params] == ptrs
    assert torch.equal(torch.cat([p.detach().reshape(-1) for p in meta.params]), ref + 1.0)


@pytest.mark.parametrize("stage", [0, 1, 2, 3])
@pytest.mark.parametrize("max_norm", [0.0, 0.05])
def test_step_matches_oracle_update(stage, max_norm):
    """Optimizer arithmetic: the surrogate loss sum(p * G_p) gives every
    parameter the gradient G_p (for stage 3 pushed through each handle's
    bucketed flatten).  The stage-3 executor's real gradients are pinned by
    test_stage3_executor_gradients_match_stage0 and, against the oracle, by
    tests/test_gpu_configs.py."""
    model = _model(1234)
    gen = torch.Generator().manual_seed(stage * 7 + int(max_norm * 100))
    names = [n for n, _ in model.named_parameters()]
    G = {n: (1e-2 * torch.randn(p.shape, generator=gen)).to(torch.bfloat16) for n, p in model.named_parameters()}
    master0 = torch.cat([p.detach().float().cpu().reshape(-1) for p in model.parameters()])
    eng = STAGES[stage](model=model, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.05)
    ref = OE.EngineRef(master0.double(), lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.05)
    for step in range(3):
        eng.zero_grad()
        eng.prepare_forward()
        if stage == 3:
            # gradients into each handle's shard through its bucketed flatten
            with eng.summon_full_params():
                params = dict(model.named_parameters())
                loss = sum((params[n] * G[n].to(DEV)).float().sum() for n in names)
                grads = torch.autograd.grad(loss, [params[n] for n in names])
                by_id = {id(params[n]): g for n, g in zip(names, grads)}
                for h in eng._handle_order:
                    h.accumulate_grad_shard([by_id[id(p)] for p in h.meta.params])
        else:
            params = dict(model.named_parameters())
            loss = sum((params[n] * G[n].to(DEV)).float().sum() for n in names)
            eng.backward(loss)
        norm = eng.step(max_grad_norm=max_norm)
        flat_g = torch.cat([G[n].double().reshape(-1) for n in names])
        rnorm = ref.step(flat_g, max_grad_norm=max_norm)
        assert abs(norm - rnorm) <= 1e-5 * rnorm
    got = torch.cat([v.reshape(-1) for v in _full_params(eng, model).values()]).double().cpu()
    if stage == 3:
        master = eng._master_all.double().cpu()
    elif stage == 0:
        master = eng.master_params.double().cpu()
    else:
        master = eng.local_master_param_shard.double().cpu()
    assert float((master - ref.master).norm() / ref.master.norm()) < 1e-5
    assert torch.equal(got.float(), master.float().to(torch.bfloat16).float())
    assert eng.step_count == 3


def _train(engine, model, steps, max_norm=0.0):
    losses = []
    for s in range(steps):
        ids = _batch(s)
        engine.zero_grad()
        engine.prepare_forward()
        loss = model(input_ids=ids, labels=ids).loss
        losses.append(float(loss.detach()))
        engine.backward(loss)
        engine.step(max_grad_norm=max_norm)
    return losses


def test_stage3_matches_stage0_training():
    m0, m3 = _model(4321), _model(4321)
    kw = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01)
    e0 = ZeROStage0DDP(model=m0, **kw)
    e3 = ZeROStage3Optimizer(model=m3, **kw)
    l0 = _train(e0, m0, 3, max_norm=0.5)
    l3 = _train(e3, m3, 3, max_norm=0.5)
    for a, b in zip(l0, l3):
        assert abs(a - b) <= 1e-2 * abs(a)
    p0, p3 = _full_params(e0, m0), _full_params(e3, m3)
    for n in p0:
        rel = float((p0[n] - p3[n]).norm() / p0[n].norm())
        assert rel < 2e-2, (n, rel)


@pytest.mark.parametrize("recompute", [True, False])
def test_stage3_matches_stage0_with_dropout(recompute):
    """zero/tests/test_zero_stages.py:195-271 at world size 1: dropout 0.2,
    torch.manual_seed before each forward; the stage-3 executor (its
    recompute restores the RNG state, so the masks replay) trains like
    stage 0: equal first-step losses, and losses and parameters within the
    bf16 bar after that."""
    kw = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01)
    m0, m3 = _model(4321, dropout=0.2), _model(4321, dropout=0.2)
    e0 = ZeROStage0DDP(model=m0, **kw)
    e3 = ZeROStage3Optimizer(model=m3, recompute=recompute, **kw)
    nodrop = float(m0.eval()(input_ids=_batch(0), labels=_batch(0)).loss.detach())
    for step in range(2):
        ids = _batch(step)
        seed = 10_000 + step * 31
        losses = []
        for m, e in ((m0, e0), (m3, e3)):
            m.train()
            e.zero_grad()
            e.prepare_forward()
            torch.manual_seed(seed)
            loss = m(input_ids=ids, labels=ids).loss
            e.backward(loss)
            e.step()
            losses.append(float(loss.detach()))
        # step 0 starts from equal weights; after it the engines' updates
        # differ in rounding (stage 0 sums the tied weight's two gradient
        # contributions in bf16, stage 3 in fp32)
        assert abs(losses[0] - losses[1]) <= (1e-6 if step == 0 else 1e-2) * abs(losses[0]), (step, losses)
        if step == 0:
            assert nodrop != losses[0]  # dropout was applied
    p0, p3 = _full_params(e0, m0), _full_params(e3, m3)
    for n in p0:
        rel = float((p0[n] - p3[n]).norm() / p0[n].norm())
        assert rel < 2e-2, (n, rel)


@pytest.mark.parametrize("recompute", [True, False])
def test_stage3_executor_gradients_match_stage0(recompute):
    """The stage-3 executor (_ShardedModuleFunction: no-grad forward, then
    recompute or the kept graph, autograd.grad per module call, bucketed
    flatten into the fp32 shard, the tied embedding/LM-head handle called
    twice) against stage 0's single autograd pass on the same kernels, on
    real batches with two micro-batches and clipping: each step starts both
    from the same master, the losses agree to 1e-6 and every parameter's
    gradient to cosine 0.99999 (stage 0 adds the tied weight's two
    contributions and the micro-batches in bf16, stage 3 in fp32)."""
    kw = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01)
    m0, m3 = _model(99), _model(99)
    e0 = ZeROStage0DDP(model=m0, **kw)
    e3 = ZeROStage3Optimizer(model=m3, recompute=recompute, **kw)
    names = [(n, p.numel()) for n, p in m0.named_parameters()]
    for step in range(3):
        e3._master_all.copy_(e0.master_params)
        if e3._param_flat is not None:
            ops.cast(e3._master_all, e3._param_flat.dtype, out=e3._param_flat)
        losses = {}
        for key, m, e in (("s0", m0, e0), ("s3", m3, e3)):
            e.zero_grad()
            e.prepare_forward()
            tot = 0.0
            for micro in range(2):
                ids = _batch(10 * step + micro)
                loss = m(input_ids=ids, labels=ids, return_logits=False).loss
                tot += float(loss.detach())
                e.backward(loss / 2)
            losses[key] = tot
        assert abs(losses["s0"] - losses["s3"]) <= 1e-6 * abs(losses["s0"])
        g0 = torch.cat([p.grad.double().reshape(-1) for p in e0.meta.params]).cpu()
        e3._finish_grads()
        g3 = e3._grad_all.double().cpu()
        off = 0
        for n, k in names:
            cos = float(torch.nn.functional.cosine_similarity(g0[off:off + k], g3[off:off + k], dim=0))
            assert cos >= 0.99999, (step, n, cos)
            off += k
        n0, n3 = e0.step(max_grad_norm=0.5), e3.step(max_grad_norm=0.5)
        assert abs(n0 - n3) <= 1e-3 * n0


def test_stage3_recompute_off_matches_recompute_on():
    """Keeping each module's forward graph gives the recompute path's
    gradients: same loss bits, same fp32 gradient flatten (up to the order of
    the embedding gradient's fp32 atomics), and the same training."""
    kw = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01)
    ma, mb = _model(55), _model(55)
    ea = ZeROStage3Optimizer(model=ma, **kw)
    eb = ZeROStage3Optimizer(model=mb, recompute=False, **kw)
    assert all(p.numel() > 0 for p in mb.parameters())
    for e, m in ((ea, ma), (eb, mb)):
        e.zero_grad()
        e.prepare_forward()
        for s in range(2):  # two micro-batches accumulate into the fp32 shard
            loss = m(input_ids=_batch(s), labels=_batch(s)).loss
            e.backward(loss)
        e._last_loss = float(loss.detach())
    assert ea._last_loss == eb._last_loss
    ea._finish_grads()
    eb._finish_grads()
    ga, gb = ea._grad_all.double(), eb._grad_all.double()
    assert float((ga - gb).norm() / ga.norm()) < 1e-5
    ea.step(max_grad_norm=0.5)
    eb.step(max_grad_norm=0.5)
    la, lb = _train(ea, ma, 3, max_norm=0.5), _train(eb, mb, 3, max_norm=0.5)
    for a, b in zip(la, lb):
        assert abs(a - b) <= 1e-4 * abs(a)
    pa, pb = _full_params(ea, ma), _full_params(eb, mb)
    for n in pa:
        assert torch.allclose(pa[n], pb[n], rtol=1e-3, atol=1e-5), n
    # parameters stay materialised and equal the bf16 rounding of the master
    assert all(p.numel() > 0 for p in mb.parameters())
    assert torch.equal(eb._param_flat, eb._master_all.to(torch.bfloat16))
    assert eb._forward_allgather_ms == 0.0


def test_block_gradients_unchanged_when_output_unused():
    """Under lzhip.functional.output_unused() (the stage-3 recompute) a
    TransformerBlock leaves its MLP's down projection unformed; the gradients
    of its input and parameters taken through that output are bit for bit
    those of the full forward, and the GEMM probe sees one launch fewer."""
    from lzhip import functional as LF

    m = _model(21)
    block = m.layers[0]
    torch.manual_seed(3)
    x0 = torch.randn(3, 64, 128, device=DEV).to(torch.bfloat16)
    dy = torch.randn(3, 64, 128, device=DEV).to(torch.bfloat16)
    params = list(block.parameters())
    res = []
    for unused in (False, True):
        x = x0.clone().requires_grad_(True)
        probe = ops.LaunchProbe()
        ops.set_gemm_probe(probe)
        try:
            if unused:
                with LF.output_unused():
                    out = block(x)
            else:
                out = block(x)
        finally:
            ops.set_gemm_probe(None)
        launches = len(probe.records)
        grads = torch.autograd.grad(out, [x] + params, grad_outputs=dy)
        res.append((grads, launches))
    for a, b in zip(res[0][0], res[1][0]):
        assert torch.equal(a, b)
    assert res[1][1] == res[0][1] - 1  # the down projection's forward product is the one launch left out


def test_stage3_recompute_off_checkpoint_restore():
    kw = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01, recompute=False)
    m_src = _model(31)
    e_src = ZeROStage3Optimizer(model=m_src, **kw)
    _train(e_src, m_src, 2, max_norm=0.25)
    m_dst = _model(32)
    e_dst = ZeROStage3Optimizer(model=m_dst, **kw)
    e_dst.load_state_dict(e_src.state_dict())
    a, b = _full_params(e_src, m_src), _full_params(e_dst, m_dst)
    for n in a:
        assert torch.equal(a[n], b[n]), n


def test_stage3_reshards_and_summons():
    model = _model(7)
    eng = ZeROStage3Optimizer(model=model, lr=1e-3, weight_decay=0.0)
    assert any(p.numel() == 0 for p in model.parameters())
    with eng.summon_full_params():
        assert all(p.numel() > 0 for p in model.parameters())
        with eng.summon_full_params():
            pass
        assert all(p.numel() > 0 for p in model.parameters())
    assert all(p.numel() == 0 for p in model.parameters())
    names = [h.name for h in eng._handle_order]
    assert names == ["tok_embeddings", "layers.0", "layers.1", "norm"]
    assert eng.handles["tok_embeddings"].module_names == ["tok_embeddings", "lm_head"]
    live, meas = eng.live_model_state_breakdown_mb(), eng.memory_state_breakdown_mb()
    for k in ("params_mb", "grads_mb", "optimizer_mb", "total_mb"):
        assert live[k] == pytest.approx(meas[k])


def test_stage3_checkpoint_restore():
    kw = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01)
    m_src = _model(2024)
    e_src = ZeROStage3Optimizer(model=m_src, **kw)
    _train(e_src, m_src, 2, max_norm=0.25)
    state = e_src.state_dict()
    m_dst = _model(9999)
    e_dst = ZeROStage3Optimizer(model=m_dst, **kw)
    e_dst.load_state_dict(state)
    assert e_dst.step_count == e_src.step_count
    a, b = _full_params(e_src, m_src), _full_params(e_dst, m_dst)
    for n in a:
        assert torch.equal(a[n], b[n]), n
    ids = _batch(7)
    for m, e in ((m_src, e_src), (m_dst, e_dst)):
        e.zero_grad()
        e.prepare_forward()
        loss = m(input_ids=ids, labels=ids).loss
        e.backward(loss)
        e.step(max_grad_norm=0.25)
    a, b = _full_params(e_src, m_src), _full_params(e_dst, m_dst)
    for n in a:
        assert torch.allclose(a[n], b[n], rtol=1e-2, atol=1e-4), n


def test_stage2_releases_full_grads_and_keeps_shard():
    model = _model(1234)
    timeline = []
    eng = ZeROStage2Optimizer(model=model, lr=1e-3, weight_decay=0.0, memory_tracker=MemoryTracker(device=DEV),
                              memory_trace_active=True, memory_state_timeline=timeline)
    ids = _batch(0)
    eng.zero_grad()
    eng.prepare_forward()
    eng.backward(model(input_ids=ids, labels=ids).loss)
    assert all(p.grad is None for p in model.parameters())
    assert eng.grad_shard is not None and float(eng.grad_shard.abs().sum()) > 0.0
    eng.step()
    assert eng.grad_shard is None and all(p.grad is None for p in model.parameters())
    labels = [t["label"] for t in timeline]
    assert labels[-3:] == ["measured_step_stage2_pre_allgather", "measured_step_stage2_post_allgather",
                           "measured_step_stage2_post_step_free_grad_shard"]
    assert timeline[-1]["live_grad_shard_mb"] == 0.0 and timeline[-1]["live_flat_grad_buffer_mb"] == 0.0
    logical, live = eng.memory_state_breakdown_mb(), eng.live_model_state_breakdown_mb()
    assert logical["grads_mb"] > 0.0 and live["grads_mb"] == 0.0


def test_stage2_grad_accumulation_matches_stage0():
    kw = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01)
    m0, m2 = _model(777), _model(777)
    e0, e2 = ZeROStage0DDP(model=m0, **kw), ZeROStage2Optimizer(model=m2, grad_bucket_numel=4096, **kw)
    for step in range(2):
        for m, e in ((m0, e0), (m2, e2)):
            e.zero_grad()
            for micro in range(2):
                ids = _batch(step * 2 + micro)
                e.backward(m(input_ids=ids, labels=ids).loss / 2)
            e.step(max_grad_norm=0.25)
    a, b = _full_params(e0, m0), _full_params(e2, m2)
    for n in a:
        assert torch.allclose(a[n], b[n], rtol=2e-2, atol=1e-3), n


@pytest.mark.parametrize("stage", [0, 1, 2, 3])
def test_tracing_labels(stage):
    model = _model(11)
    coll = TracingCollectives(LocalCollectives())
    eng = STAGES[stage](model=model, lr=1e-3, collectives=coll)
    ids = _batch(0)
    eng.zero_grad()
    eng.prepare_forward()
    eng.backward(model(input_ids=ids, labels=ids).loss)
    eng.step()
    labels = {r["label"] for r in coll.consume_trace()}
    expect = {
        0: "stage0.step.allreduce.grad_bucket",
        1: "stage1.step.allgather.updated_param_shard",
        2: "stage2.backward.reduce_scatter.flat_grad_buffer",
        3: "stage3.backward.reduce_scatter.layers.0",
    }[stage]
    assert expect in labels, labels
    if stage == 3:
        assert "stage3.forward.allgather.tok_embeddings" in labels


def test_engine_state_dict_round_trip_stage1():
    kw = dict(lr=1e-3, weight_decay=0.1)
    m = _model(5)
    e = ZeROStage1Optimizer(model=m, **kw)
    _train(e, m, 2)
    st = e.state_dict()
    assert {"step_count", "shard_start", "shard_end", "local_master_param_shard", "exp_avg", "exp_avg_sq"} <= set(st)
    m2 = _model(6)
    e2 = ZeROStage1Optimizer(model=m2, **kw)
    e2.load_state_dict(st)
    for (n, a), (_, b) in zip(m.named_parameters(), m2.named_parameters()):
        assert torch.equal(a, b), n
