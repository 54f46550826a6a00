"""Host-side logic of the product, checked on the CPU (no GPU compute):
index maps against the oracle, configs, data streams, profiler helpers,
collective tracing, CLI flags, the C-ABI export table and the refusal to
compute on CPU tensors."""
from __future__ import annotations

import ctypes
import re
import time
from pathlib import Path

import pytest
import torch

from oracle import data as OD
from oracle import flat as OF
from oracle import model as OM

ROOT = Path(__file__).resolve().parents[1]


def _ocfg(cfg) -> OM.Cfg:
    return OM.Cfg(vocab_size=cfg.vocab_size, dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.n_heads,
                  n_kv_heads=cfg.n_kv_heads, ffn_dim=cfg.ffn_dim, rope_theta=cfg.rope_theta,
                  tie_word_embeddings=cfg.tie_word_embeddings)


# ---------------------------------------------------------------------------
# model construction and index maps
# ---------------------------------------------------------------------------

def test_presets_scale_monotonically():
    from model import build_medium_config, build_small_config, build_tiny_config, estimate_num_parameters

    t, s, m = (estimate_num_parameters(b()) for b in (build_tiny_config, build_small_config, build_medium_config))
    assert t < s < m
    assert 40_000_000 <= t <= 60_000_000
    assert 250_000_000 <= s <= 400_000_000
    assert 1_100_000_000 <= m <= 1_500_000_000


@pytest.mark.parametrize("size,count", [("plumbing", 11_094_272), ("125m", 100_092_672), ("1b", 820_578_304),
                                        ("7b", 5_802_037_248)])
def test_benchmark_presets(size, count):
    from model import build_config, estimate_num_parameters

    cfg = build_config(size, vocab_size=32000)
    assert cfg.rope_theta == 10_000.0
    assert estimate_num_parameters(cfg) == count == OM.num_parameters(_ocfg(cfg))


def test_config_validation_errors():
    from model import ModelConfig

    with pytest.raises(ValueError):
        ModelConfig(name="x", vocab_size=10, max_seq_len=8, dim=30, n_layers=1, n_heads=4, n_kv_heads=2)
    with pytest.raises(ValueError):
        ModelConfig(name="x", vocab_size=10, max_seq_len=8, dim=32, n_layers=1, n_heads=4, n_kv_heads=3)
    cfg = ModelConfig(name="x", vocab_size=10, max_seq_len=8, dim=320, n_layers=1, n_heads=10, n_kv_heads=2)
    assert cfg.ffn_dim == 1024 and cfg.with_vocab_size(99).vocab_size == 99


def test_init_matches_oracle_rng_order():
    """Same seed -> identical initial weights as the oracle's restatement of
    the reference construction order (pinned by the golden loss)."""
    from model import LlamaForCausalLM, ModelConfig

    cfg = ModelConfig(name="unit_test", vocab_size=128, max_seq_len=16, dim=64, n_layers=2, n_heads=4, n_kv_heads=2,
                      ffn_dim=128)
    torch.manual_seed(123)
    model = LlamaForCausalLM(cfg)
    torch.manual_seed(123)
    P = OM.init_params(_ocfg(cfg))
    sd = model.state_dict()
    assert set(sd) - {"lm_head.weight"} == set(P)
    for k, v in P.items():
        assert torch.equal(sd[k], v), k
    assert model.lm_head.weight is model.tok_embeddings.weight


@pytest.mark.parametrize("size", ["plumbing", "125m", "1b", "7b"])
def test_flat_metadata_bit_exact(size):
    from model import LlamaForCausalLM, build_config
    from zero.common import build_flat_param_metadata

    cfg = build_config(size, vocab_size=32000)
    with torch.device("meta"):
        model = LlamaForCausalLM(cfg)
    meta = build_flat_param_metadata(model)
    specs = OM.param_specs(_ocfg(cfg))
    offs, numels, total = OF.flat_layout([s for _, s in specs])
    assert meta.total_numel == total
    assert meta.offsets == [int(o) for o in offs]
    assert [tuple(s) for s in meta.shapes] == [s for _, s in specs]
    names = {id(p): n for n, p in model.named_parameters()}
    assert [names[id(p)] for p in meta.params] == [n for n, _ in specs]


@pytest.mark.parametrize("size", ["plumbing", "1b"])
def test_stage3_handle_plan_matches_oracle(size):
    from model import LlamaForCausalLM, build_config
    from zero.stage3_optimizer import plan_handles

    cfg = build_config(size, vocab_size=32000)
    with torch.device("meta"):
        model = LlamaForCausalLM(cfg)
    names = {id(p): n for n, p in model.named_parameters()}
    plan = plan_handles(model)
    ref = OF.stage3_handles(_ocfg(cfg))
    assert [p[0] for p in plan] == [h["name"] for h in ref]
    assert [p[1] for p in plan] == [h["module_names"] for h in ref]
    assert [[names[id(x)] for x in p[2]] for p in plan] == [h["params"] for h in ref]


def test_shard_and_bucket_maps_match_oracle():
    from zero.common import bucket_ranges, compute_shard_spec

    for total in (1, 7, 26, 820_578_304, 5_802_037_248):
        for ws in (1, 2, 3, 8):
            for r in range(ws):
                s = compute_shard_spec(total, r, ws)
                ref = OF.shard_spec(total, r, ws)
                assert (s.shard_start, s.shard_end, s.shard_numel, s.chunk_size) == (
                    ref["shard_start"], ref["shard_end"], ref["shard_numel"], ref["chunk_size"])
        assert bucket_ranges(0, total) == OF.bucket_plan(total)


def test_product_refuses_cpu_compute():
    from lzhip import ops
    from model import LlamaForCausalLM, ModelConfig

    cfg = ModelConfig(name="t", vocab_size=32, max_seq_len=8, dim=32, n_layers=1, n_heads=2, n_kv_heads=1, ffn_dim=64)
    model = LlamaForCausalLM(cfg)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        model(torch.zeros(1, 8, dtype=torch.long))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.rmsnorm_fwd(torch.zeros(2, 8), torch.ones(8), 1e-5)


# ---------------------------------------------------------------------------
# data
# ---------------------------------------------------------------------------

def test_synthetic_pattern_matches_oracle():
    from data import SyntheticPatternDataset

    it = iter(SyntheticPatternDataset(seq_len=8, vocab_size=13))
    ref = next(OD.ramp_chunks(8, 13, 3))
    got = torch.stack([next(it) for _ in range(3)])
    assert torch.equal(got, ref)


def test_synthetic_uniform_matches_oracle():
    from data import SyntheticUniformDataset

    ds = SyntheticUniformDataset(seq_len=127, vocab_size=32000, seed=0)
    it = iter(ds)
    got = torch.stack([next(it) for _ in range(4)])
    ref = next(OD.uniform_chunks(127, 32000, 4, seed=0))
    assert torch.equal(got, ref)
    assert int(got.min()) >= 0 and int(got.max()) < 32000


def test_rank_shard_and_packed_dataset():
    from data import PackedFineWebDataset, RankShardIterableDataset, SyntheticPatternDataset

    base = SyntheticPatternDataset(seq_len=4, vocab_size=97, num_sequences=6)
    r1 = list(RankShardIterableDataset(base, rank=1, world_size=2))
    assert len(r1) == 3 and torch.equal(r1[0], list(base)[1])
    with pytest.raises(ValueError):
        RankShardIterableDataset(base, rank=2, world_size=2)

    class Tok:
        def encode(self, text, add_special_tokens=False):
            return [ord(c) % 32 for c in text]

    docs = [{"text": "abcd"}, {"text": ""}, "efgh", {"text": "ijklmnopq"}]
    chunks = list(PackedFineWebDataset(docs, Tok(), 4, eos_token_id=1))
    # the concatenation of the non-empty documents, each followed by EOS, cut
    # into [5] chunks; the remainder is held back
    stream = []
    for t in ("abcd", "efgh", "ijklmnopq"):
        stream += [ord(c) % 32 for c in t] + [1]
    n = len(stream) // 5
    assert len(chunks) == n and all(c.shape == (5,) and c.dtype == torch.long for c in chunks)
    assert torch.equal(torch.stack(chunks).reshape(-1), torch.tensor(stream[:5 * n]))


def test_token_packer_and_offline_fineweb():
    from data import FineWebUnavailable, TokenPacker, load_fineweb_stream, load_llama_tokenizer

    p = TokenPacker(3)
    assert p.push([]) == []
    assert p.push([1, 2]) == []
    out = p.push(list(range(3, 11)))  # 1..10 so far: chunks [1,2,3] [4,5,6] [7,8,9], 10 held
    assert [c.tolist() for c in out] == [[1, 2, 3], [4, 5, 6], [7, 8, 9]]
    assert [c.tolist() for c in p.push([11, 12])] == [[10, 11, 12]]
    with pytest.raises(ValueError):
        TokenPacker(0)
    with pytest.raises(FineWebUnavailable, match="synthetic"):
        load_llama_tokenizer("meta-llama/Llama-3.1-8B")
    with pytest.raises(FineWebUnavailable):
        load_fineweb_stream("sample-10BT")


# ---------------------------------------------------------------------------
# profiler
# ---------------------------------------------------------------------------

def test_profiler_helpers():
    from model import build_config, build_tiny_config
    from profiler import (
        MemoryTracker,
        TimerRegistry,
        estimate_transformer_train_flops,
        flops_to_tflops_per_second,
        overlap_efficiency,
    )

    assert overlap_efficiency(step_ms=15.0, compute_ms=10.0, communication_ms=5.0) == 0.0
    assert overlap_efficiency(step_ms=10.0, compute_ms=10.0, communication_ms=5.0) == 1.0
    reg = TimerRegistry(device=None)
    t = reg.timer("sleep")
    t.start()
    time.sleep(0.01)
    assert t.stop() >= 10.0
    assert reg.summarize()["sleep"].count == 1 and reg.summarize()["sleep"].total_ms > 0
    with pytest.raises(RuntimeError):
        t.stop()
    for ms in (1.0, 2.0, 3.0, 4.0):  # summary statistics over known samples
        t._done_ms.append(ms)
    s = reg.timer("sleep").summary()
    assert s.count == 5 and s.min_ms == 1.0 and s.max_ms >= 10.0
    assert s.p50_ms == 3.0 and abs(s.mean_ms - s.total_ms / 5) < 1e-12
    # nearest rank with round() (reference profiler/timer.py:62-64), not interpolation:
    # two samples give p50 = the first (round(0.5) == 0); p95 of 20 is sample 18 (round(18.05))
    two = reg.timer("two")
    two._done_ms.extend([1.0, 2.0])
    assert two.summary().p50_ms == 1.0 and two.summary().p95_ms == 2.0
    twenty = reg.timer("twenty")
    twenty._done_ms.extend([float(i * i) for i in range(20)])
    assert twenty.summary().p95_ms == 18.0 * 18.0 and twenty.summary().p50_ms == 10.0 * 10.0
    mt = MemoryTracker(device=None)
    mt.record("before")
    mt.record("after")
    assert [s["label"] for s in mt.as_dicts()] == ["before", "after"]
    cfg = build_tiny_config(vocab_size=1024, max_seq_len=64)
    s0 = estimate_transformer_train_flops(cfg, batch_size=4, seq_len=64, grad_accum_steps=2, world_size=4, stage=0)
    s3 = estimate_transformer_train_flops(cfg, batch_size=4, seq_len=64, grad_accum_steps=2, world_size=4, stage=3)
    assert 0 < s0 < s3 and abs(s3 / s0 - 4 / 3) < 1e-12
    assert flops_to_tflops_per_second(1e12, 0.5) == 2.0
    # workload figures: 1B at B=8, S=2048: 93.884 TFLOP (3x) / 125.179 (4x); 125M at B=16, S=1024: 11.702
    one_b = build_config("1b", vocab_size=32000)
    assert abs(estimate_transformer_train_flops(one_b, 8, 2048) / 1e12 - 93.884) < 5e-3
    assert abs(estimate_transformer_train_flops(one_b, 8, 2048, stage=3) / 1e12 - 125.179) < 5e-3
    m125 = build_config("125m", vocab_size=32000)
    assert abs(estimate_transformer_train_flops(m125, 16, 1024) / 1e12 - 11.702) < 5e-3


# ---------------------------------------------------------------------------
# collectives
# ---------------------------------------------------------------------------

def test_tracing_collectives_records():
    from collectives import LocalCollectives, TracingCollectives
    from train_zero import aggregate_collective_trace

    traced = TracingCollectives(LocalCollectives())
    shard = torch.arange(4, dtype=torch.bfloat16)
    with traced.label_scope("stage2.step.allgather.updated_param_shard"):
        gathered = traced.allgather(shard)
    rec = traced.consume_trace()
    assert gathered.numel() == 4 and gathered.data_ptr() != shard.data_ptr()
    assert len(rec) == 1 and rec[0]["op"] == "allgather"
    assert rec[0]["label"] == "stage2.step.allgather.updated_param_shard"
    assert rec[0]["input_bytes"] == 8 and rec[0]["output_bytes"] == 8
    assert traced.consume_trace() == []
    summary = aggregate_collective_trace([
        {"op": "allgather", "label": "a", "elapsed_ms": 2.0, "input_bytes": 4, "output_bytes": 16},
        {"op": "allgather", "label": "a", "elapsed_ms": 3.0, "input_bytes": 4, "output_bytes": 16},
        {"op": "reduce_scatter", "label": "b", "elapsed_ms": 1.5, "input_bytes": 16, "output_bytes": 4},
    ])
    assert summary[0] == {"op": "allgather", "label": "a", "calls": 2, "elapsed_ms": 5.0, "input_bytes": 8.0,
                          "output_bytes": 32.0}
    local = LocalCollectives()
    x = torch.ones(3)
    assert local.allreduce_inplace(x) is x
    assert local.is_identity and not traced.is_identity


def test_multiprocess_collectives_are_rejected():
    from collectives import SendRecvCollectives, TorchCollectives

    for cls in (SendRecvCollectives, TorchCollectives):
        with pytest.raises(RuntimeError, match="world_size=1"):
            cls()


# ---------------------------------------------------------------------------
# CLI
# ---------------------------------------------------------------------------

def test_cli_defaults_match_reference():
    import train
    import train_zero

    a = train.parse_args([])
    assert (a.model_size, a.seq_len, a.batch_size, a.grad_accum_steps, a.max_steps) == ("tiny", 512, 2, 8, 200)
    assert (a.learning_rate, a.weight_decay, a.beta1, a.beta2, a.max_grad_norm) == (3e-4, 0.1, 0.9, 0.95, 1.0)
    assert (a.dtype, a.device, a.seed, a.loss_chunk_size, a.data_mode) == ("bfloat16", "cuda", 1337, 128, "fineweb")
    z = train_zero.parse_args([])
    assert (z.zero_stage, z.collective_impl, z.dtype, z.max_grad_norm, z.data_mode) == (0, "torch", "float32", 0.0,
                                                                                         "synthetic")
    assert z.stage2_grad_bucket_mb == 64.0 and z.grad_bucket_numel == 25_000_000 and z.synthetic_vocab_size == 8192
    z = train_zero.parse_args(["--zero-stage", "3", "--model-size", "1b", "--data-mode", "synthetic-uniform"])
    assert z.zero_stage == 3 and z.model_size == "1b"


def test_step_line_matches_harness_regex():
    """The stdout step line format the reference harness parses
    (experiments/harness.py:26-28)."""
    line = ("[step 00010] loss=5.1234 avg100=5.4321 tokens/s=123,456 grad_norm=0.812 "
            "fb_ms=10.00 comm_ms=0.00 opt_ms=1.23 tflops=123.456")
    pat = re.compile(r"\[step\s+(\d+)\]\s+loss=([0-9.]+).*tokens/s=([0-9,]+)")
    assert pat.search(line)


# ---------------------------------------------------------------------------
# C ABI
# ---------------------------------------------------------------------------

def _declared_symbols():
    text = (ROOT / "include" / "llamazero_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lz_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import lzhip._lib as L

    if not L.LIB_PATH.exists():
        pytest.skip("libllamazero_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(L.LIB_PATH))
    declared = _declared_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert set(declared) == set(L.SIGNATURES)
    assert lib.lz_version() == 1


def test_adamw_norm_workspace_size():
    """One float64 partial per 128-thread AdamW workgroup (4 elements per
    thread) plus the 256 second-level sums; host arithmetic only."""
    import lzhip._lib as L

    if not L.LIB_PATH.exists():
        pytest.skip("libllamazero_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(L.LIB_PATH))
    fn = lib.lz_adamw_norm_workspace
    fn.restype, fn.argtypes = ctypes.c_int64, [ctypes.c_int64]
    assert fn(0) == 0
    for n in (1, 3, 4, 511, 512, 513, 1_100_048_384):
        assert fn(n) == -(-(n // 4) // 128) + 256


def test_library_defines_every_kernel_launch_stub():
    """Every kernel the library launches has its host launch stub: an undefined
    __device_stub__ symbol would only fail when the library is loaded."""
    import shutil
    import subprocess

    import lzhip._lib as L

    if not L.LIB_PATH.exists():
        pytest.skip("libllamazero_hip.so not built (run __graft_entry__.build())")
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-C", "--undefined-only", str(L.LIB_PATH)], capture_output=True, text=True, check=True)
    stubs = [line for line in out.stdout.splitlines() if "__device_stub__" in line]
    assert not stubs, stubs[:5]


def test_gemm_plan_codes_and_workspace():
    """lz_gemm_plan (host only, no launch): 64 * cfg + splits with a known
    kernel configuration and 1..32 splits; the workspace is splits x M x N
    fp32 exactly when the product is split; the benchmark decodes the same
    names.  Weight gradients over 16384 tokens split, the 1B forward does
    not."""
    import lzhip._lib as L
    from lzhip import ops

    if not L.LIB_PATH.exists():
        pytest.skip("libllamazero_hip.so not built (run __graft_entry__.build())")
    lib = L.load()
    shapes = [(4096, 2048, 16384, 0, 0), (768, 768, 16384, 0, 0), (32000, 768, 16384, 0, 0),
              (16384, 2048, 5632, 1, 0), (16384, 4096, 2048, 1, 1), (16384, 1280, 768, 1, 1), (1000, 1000, 520, 0, 1),
              (16384, 768, 768, 1, 1), (16384, 768, 4096, 1, 0), (16384, 768, 32000, 1, 0)]
    prefix = {5: "gemm_dma_kernel<", 6: "gemm_dma_n192_kernel<"}
    for M, N, K, ak, bk in shapes:
        code = int(lib.lz_gemm_plan(M, N, K, ak, bk))
        cfg, splits = code // 64, code % 64
        assert cfg in (0, 1, 2, 5, 6) and 1 <= splits <= 32, (M, N, K, code)
        assert cfg != 6 or (ak and splits == 1), (M, N, K, code)  # 256x192 tiles: K-major A, unsplit
        ws = int(lib.lz_gemm_workspace(M, N, K, ak, bk))
        assert ws == (splits * M * N * 4 if splits > 1 else 0), (M, N, K, splits, ws)
        name = ops.gemm_kernel_name((bool(ak), bool(bk), code))
        assert name.startswith(prefix.get(cfg, "gemm_kernel<"))
        assert ("split-K x%d" % splits in name) == (splits > 1)
    assert int(lib.lz_gemm_plan(768, 768, 16384, 0, 0)) % 64 > 8  # the 125M weight gradient splits widely
    assert int(lib.lz_gemm_plan(16384, 4096, 2048, 1, 1)) == 5 * 64 + 1
    # at 16384 rows, N = 768 fills 256 CUs with 256x192 tiles (3 x 64 tiles of 256 would leave 64 idle); N = 1280
    # keeps 256x256 (a short second round of 64 tiles beats a 3/4-full one of 192), and so do the 1B model's
    # N = 2048 products (512 tiles: two full rounds)
    for N, K, bk in ((768, 768, 1), (768, 2048, 1), (768, 768, 0), (768, 1280, 0), (768, 4096, 0), (768, 32000, 0)):
        assert int(lib.lz_gemm_plan(16384, N, K, 1, bk)) == 6 * 64 + 1, (N, K, bk)
    for N, K, bk in ((1280, 768, 1), (2048, 2048, 1), (2048, 5632, 1), (32000, 2048, 1), (32000, 768, 1),
                     (2048, 2048, 0), (2048, 32000, 0)):
        assert int(lib.lz_gemm_plan(16384, N, K, 1, bk)) // 64 == 5, (N, K, bk)
    # an M/N-major operand's split (K rows of ld >= M or N) stays under 2^30 elements: the 7B model's weight
    # gradients over 64 and 128 sequences of 2048 split at least 2-6 ways
    for M, N, K, least in ((22016, 4096, 131072, 3), (4096, 11008, 131072, 2), (22016, 4096, 262144, 6),
                           (4096, 11008, 262144, 3), (8192, 512, 262144, 3)):
        code = int(lib.lz_gemm_plan(M, N, K, 0, 0))
        assert code // 64 == 5 and code % 64 >= least, (M, N, K, code)
        kper = -(-(-(-K // (code % 64))) // 64) * 64
        assert kper * max(M, N) + 256 < 1 << 30, (M, N, K, code)
    assert int(lib.lz_gemm_plan(0, 10, 10, 1, 1)) == 0


def test_loss_scaler_follows_torch_grad_scaler():
    """lzhip.optim.LossScaler's schedule (reference train.py:213-214,254-269:
    torch.cuda.amp.GradScaler) against torch.amp.GradScaler itself on the
    CPU: the same scale after every step for a pattern of overflowing and
    finite steps, the same steps skipped, growth after growth_interval
    finite steps, backoff on overflow; disabled it is the identity."""
    from lzhip.optim import LossScaler

    class _Opt:
        def __init__(self):
            self.steps = 0
            self.discarded = 0

        def step(self):
            self.steps += 1

        def discard_step(self):
            self.discarded += 1

    pattern = [False, True, False, False, False, True, True, False, False, False, False, False]
    p = torch.nn.Parameter(torch.zeros(3))
    topt = torch.optim.SGD([p], lr=1.0)
    ts = torch.amp.GradScaler("cpu", init_scale=1024.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=3)
    ls = LossScaler(init_scale=1024.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=3)
    fake = _Opt()
    torch_steps = 0
    ts.scale(torch.ones(()))  # torch's scaler creates its scale on first use
    for overflow in pattern:
        topt.zero_grad()
        p.grad = torch.full((3,), float("inf") if overflow else 1.0)
        before = p.detach().clone()
        ts.step(topt)
        ts.update()
        torch_steps += int(not torch.equal(before, p.detach()))
        ls.step(fake, float("inf") if overflow else 1.0)
        ls.update()
        assert ls.scale_value() == ts.get_scale()
    assert fake.steps == torch_steps == pattern.count(False)
    assert fake.discarded == pattern.count(True)
    restored = LossScaler()
    restored.load_state_dict(ls.state_dict())
    assert restored.scale_value() == ls.scale_value() and restored.state_dict() == ls.state_dict()
    off = LossScaler(enabled=False)
    off.step(fake, float("nan"))  # disabled: the step runs whatever the norm
    off.update()
    assert off.scale_value() == 1.0 and fake.steps == torch_steps + 1 and off.state_dict() == {}


def test_fit_sweep_stops_at_the_first_out_of_memory():
    """bench.py's 7B fit sweep doubles the micro-batch until a size runs out
    of device memory: that size is recorded as {"oom": True} and the sweep
    ends; the sizes before it keep their rows, and errors other than
    out-of-memory are not swallowed (host logic only: the run is a stub)."""
    import bench

    seen = []

    def run_one(b):
        seen.append(b)
        if b == 8:
            raise torch.cuda.OutOfMemoryError("stub: out of memory")
        return {"micro_batch": b, "tokens_per_s": 1.0}

    rows = bench.sweep_batches(run_one, 64)
    assert seen == [1, 2, 4, 8]
    assert rows[:3] == [{"micro_batch": b, "tokens_per_s": 1.0} for b in (1, 2, 4)]
    assert rows[3] == {"micro_batch": 8, "oom": True}
    assert [r["micro_batch"] for r in bench.sweep_batches(lambda b: {"micro_batch": b}, 5)] == [1, 2, 4]

    def broken(b):
        raise ValueError("not a memory error")

    with pytest.raises(ValueError):
        bench.sweep_batches(broken, 4)
