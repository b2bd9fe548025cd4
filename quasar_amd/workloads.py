"""The five sampler workloads, as synthetic batches of 151,936-wide fp32 logit rows.

Each workload fixes the logit distribution, the sampler parameters (passed as float32,
like the reference's ``quasar_sampler_config``), the preloaded history and a workload
seed.  Logits, history ids and per-row sampler seeds are pure functions of
(seed, row, column) computed by the portable generator in ``csrc/qs_gen.h``, so the GPU
and the host produce the same bits for any row.

``peaked_b256`` is the throughput workload: batch 256, peaked rows
(N(0, 1.5) plus +12 at one column per row), repeat penalty 1.1 over a 256-id history,
temperature 0.8, top-k 40, top-p 0.95, min-p 0.05.
"""
from dataclasses import dataclass, replace

VOCAB = 151936

DIST_NORMAL, DIST_NORMAL_PEAK, DIST_STUDENT_T3 = 0, 1, 2


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    dist: int
    sigma: float
    boost: float
    temperature: float
    top_p: float
    top_k: int
    min_p: float
    repeat_penalty: float
    repeat_last_n: int      # ring capacity (sample.h's repeat_last_n)
    hist_len: int           # ids preloaded into the ring before the first pick
    hist_pool: int          # >0: history drawn from a per-row pool of this many ids
    seed: int
    vocab: int = VOCAB
    description: str = ""

    def params(self):
        """(temperature, top_p, top_k, min_p, repeat_penalty, repeat_last_n)."""
        return (self.temperature, self.top_p, self.top_k, self.min_p, self.repeat_penalty,
                self.repeat_last_n)

    def with_batch(self, batch):
        return replace(self, batch=batch)

    def algorithmic_bytes_per_row(self):
        """Logits read once, history ids read once, one id written, u64 RNG state read and
        written: 4V + 4H + 4 + 16."""
        return 4 * self.vocab + 4 * self.hist_len + 4 + 16


WORKLOADS = {
    "greedy_b1": Workload(
        "greedy_b1", 1, DIST_NORMAL, 2.0, 0.0, 0.0, 1.0, 0, 0.0, 1.0, 0, 0, 0, 0xC1,
        description="greedy argmax (temperature 0), batch 1, N(0, 2.0)"),
    "full_b1": Workload(
        "full_b1", 1, DIST_NORMAL, 2.0, 0.0, 0.7, 0.9, 40, 0.05, 1.1, 64, 64, 0, 0xC2,
        description="full sampler, batch 1, N(0, 2.0), penalty 1.1 over 64 uniform ids, "
                    "T 0.7, top-k 40, top-p 0.9, min-p 0.05"),
    "peaked_b256": Workload(
        "peaked_b256", 256, DIST_NORMAL_PEAK, 1.5, 12.0, 0.8, 0.95, 40, 0.05, 1.1, 256, 256,
        0, 0xC3,
        description="batched full sampler, batch 256, N(0, 1.5) + 12 at one column per row, "
                    "penalty 1.1 over 256 ids, T 0.8, top-k 40, top-p 0.95, min-p 0.05"),
    "studentt_b1024": Workload(
        "studentt_b1024", 1024, DIST_STUDENT_T3, 2.0, 0.0, 1.0, 0.9, 0, 0.0, 1.0, 0, 0, 0,
        0xC4,
        description="top-k disabled, batch 1024, 2.0 * Student-t(3), T 1.0, top-p 0.9, "
                    "no min-p, no penalty"),
    "large_b4096": Workload(
        "large_b4096", 4096, DIST_NORMAL, 2.0, 0.0, 0.6, 0.95, 200, 0.02, 1.3, 512, 512, 256,
        0xC5,
        description="batch 4096, N(0, 2.0), penalty 1.3 over 512 ids drawn from a 256-id "
                    "pool (duplicates), T 0.6, top-k 200, top-p 0.95, min-p 0.02"),
}

# Beyond the five workloads: settings that exercise the general nucleus path.
STRESS = {
    "nucleus_b8": Workload(
        "nucleus_b8", 8, DIST_NORMAL, 2.0, 0.0, 1.0, 0.9, 0, 0.0, 1.0, 0, 0, 0, 0xD1,
        description="top-k off, top-p 0.9 over N(0, 2.0) at T 1: nucleus of ~36k ids"),
    "fullwindow_b8": Workload(
        "fullwindow_b8", 8, DIST_NORMAL, 1.0, 0.0, 1.0, 1.0, 0, 0.0, 1.0, 0, 0, 0, 0xD2,
        description="every cut disabled: draw over the whole 30-nat window"),
    "minp_only_b8": Workload(
        "minp_only_b8", 8, DIST_NORMAL, 2.0, 0.0, 1.0, 1.0, 0, 0.1, 1.2, 64, 64, 0, 0xD3,
        description="top-k and top-p off, min-p 0.1, penalty 1.2"),
    "peaked_tail_b64": Workload(
        "peaked_tail_b64", 64, DIST_NORMAL_PEAK, 2.0, 30.0, 1.0, 1.0, 300, 0.0, 1.0, 0, 0, 0,
        0xD4,
        description="one column 30 above N(0, 2.0), top-k 300, top-p and min-p off: the "
                    "draw sums 300 probabilities, most of them below 2^-29"),
}

BENCH_WORKLOAD = "peaked_b256"
