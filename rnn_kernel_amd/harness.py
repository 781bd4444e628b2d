"""Training-speed harness for the GRU path: the reference's benchmark loop
(rnn_benchmark.py) for this package's GRU, with its model, step, timing
breakdown and CSV schema.

Reference behaviour kept:
* model = recurrent layer(s) + Linear(hidden_size, 1) head, prediction
  [B, T] (rnn_benchmark.py:510,525); with ``sequence_chunk_len`` > 0 the
  sequence runs in chunks carrying the hidden state, without detaching
  (:513-520);
* data = ``dataset_batches`` random (x [B,T,I], y [B,T]) pairs, x and y
  ~ N(0,1) (:610-620), cycled through warm-up and timed steps (:725-742);
* step = zero_grad(set_to_none) -> forward -> MSE -> backward -> AdamW
  (lr, weight_decay=1e-4) (:628-639,722); the optional breakdown records
  each phase with events (:642-675);
* one CSV row per hidden size with the reference's columns (:874-905).

Here the head, loss and optimiser are this package's HIP versions
(``LinearHead``, ``mse_loss``, ``AdamW``) by default; ``--torch-ops`` uses
PyTorch's (nn.Linear, F.mse_loss, torch.optim.AdamW) around the same GRU.

    python -m rnn_kernel_amd.harness --hidden-sizes 256 --batch-size 64 \\
        --seq-len 512 --input-dim 256 --num-layers 1 --output-csv out.csv
"""
from __future__ import annotations

import argparse
import csv
import gc
import time
from dataclasses import asdict, dataclass
from typing import Iterable, List, Optional

import torch
import torch.nn.functional as F
from torch import nn

from .gru import GRU, check_recurrences
from .train import AdamW, LinearHead, mse_loss

IMPLEMENTATION = "rnn_kernel_amd"

# Column order of the reference's results CSV (rnn_benchmark.py:874-899).
CSV_FIELDS = [
    "cell_type",
    "implementation",
    "hidden_size",
    "sequence_chunk_len",
    "a100_block_threads",
    "deterministic",
    "cudnn_enabled",
    "cudnn_benchmark",
    "cuda_matmul_allow_tf32",
    "cudnn_allow_tf32",
    "compile_model",
    "params",
    "ms_per_step",
    "zero_grad_ms_per_step",
    "forward_ms_per_step",
    "loss_ms_per_step",
    "backward_ms_per_step",
    "optimizer_ms_per_step",
    "measured_ms_per_step",
    "steps_per_second",
    "tokens_per_second",
    "peak_memory_gb",
    "last_loss",
    "status",
]


@dataclass
class StepTiming:
    zero_grad_ms: float
    forward_ms: float
    loss_ms: float
    backward_ms: float
    optimizer_ms: float

    @property
    def measured_ms(self) -> float:
        return self.zero_grad_ms + self.forward_ms + self.loss_ms + self.backward_ms + self.optimizer_ms


@dataclass
class BenchmarkResult:
    cell_type: str
    implementation: str
    hidden_size: int
    sequence_chunk_len: int
    a100_block_threads: int
    deterministic: bool
    cudnn_enabled: bool
    cudnn_benchmark: bool
    cuda_matmul_allow_tf32: bool
    cudnn_allow_tf32: bool
    compile_model: bool
    params: int
    ms_per_step: Optional[float]
    zero_grad_ms_per_step: Optional[float]
    forward_ms_per_step: Optional[float]
    loss_ms_per_step: Optional[float]
    backward_ms_per_step: Optional[float]
    optimizer_ms_per_step: Optional[float]
    measured_ms_per_step: Optional[float]
    steps_per_second: Optional[float]
    tokens_per_second: Optional[float]
    peak_memory_gb: Optional[float]
    last_loss: Optional[float]
    status: str


class BenchmarkModel(nn.Module):
    """GRU stack + Linear(hidden, 1) head; forward(x [B,T,I]) -> pred [B,T]."""

    def __init__(self, input_dim: int, hidden_size: int, num_layers: int, sequence_chunk_len: int = 0,
                 torch_ops: bool = False) -> None:
        super().__init__()
        self.rnn = GRU(input_dim, hidden_size, num_layers=num_layers, batch_first=True)
        self.head = nn.Linear(hidden_size, 1) if torch_ops else LinearHead(hidden_size)
        self.torch_ops = torch_ops
        self.sequence_chunk_len = int(sequence_chunk_len)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.sequence_chunk_len > 0 and x.size(1) > self.sequence_chunk_len:
            outputs = []
            hidden = None
            for start in range(0, x.size(1), self.sequence_chunk_len):
                out, hidden = self.rnn(x[:, start:start + self.sequence_chunk_len, :], hidden)
                outputs.append(out)
            out = torch.cat(outputs, dim=1)
        else:
            out, _ = self.rnn(x)
        pred = self.head(out)
        return pred.squeeze(-1) if self.torch_ops else pred


def count_parameters(model: nn.Module) -> int:
    return sum(p.numel() for p in model.parameters())


def make_random_batches(num_batches: int, batch_size: int, seq_len: int, input_dim: int, device):
    return [(torch.randn(batch_size, seq_len, input_dim, device=device),
             torch.randn(batch_size, seq_len, device=device)) for _ in range(num_batches)]


def _loss_fn(torch_ops: bool):
    return F.mse_loss if torch_ops else mse_loss


def train_step(model, optimizer, x, y, loss_fn) -> torch.Tensor:
    optimizer.zero_grad(set_to_none=True)
    pred = model(x)
    loss = loss_fn(pred, y)
    loss.backward()
    optimizer.step()
    return loss.detach()


def timed_train_step(model, optimizer, x, y, loss_fn, device):
    events = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
    events[0].record()
    optimizer.zero_grad(set_to_none=True)
    events[1].record()
    pred = model(x)
    events[2].record()
    loss = loss_fn(pred, y)
    events[3].record()
    loss.backward()
    events[4].record()
    optimizer.step()
    events[5].record()
    torch.cuda.synchronize(device)
    timing = StepTiming(*(events[i].elapsed_time(events[i + 1]) for i in range(5)))
    return loss.detach(), timing


def run_case(hidden_size: int, batches, args, device) -> BenchmarkResult:
    model = BenchmarkModel(args.input_dim, hidden_size, args.num_layers, args.sequence_chunk_len,
                           torch_ops=args.torch_ops).to(device)
    params = count_parameters(model)
    opt_cls = torch.optim.AdamW if args.torch_ops else AdamW
    optimizer = opt_cls(model.parameters(), lr=args.lr, weight_decay=1e-4)
    loss_fn = _loss_fn(args.torch_ops)
    common = dict(
        cell_type="GRU", implementation=IMPLEMENTATION + ("+torch_ops" if args.torch_ops else ""),
        hidden_size=hidden_size, sequence_chunk_len=args.sequence_chunk_len, a100_block_threads=0,
        deterministic=args.deterministic, cudnn_enabled=torch.backends.cudnn.enabled,
        cudnn_benchmark=torch.backends.cudnn.benchmark,
        cuda_matmul_allow_tf32=torch.backends.cuda.matmul.allow_tf32,
        cudnn_allow_tf32=torch.backends.cudnn.allow_tf32, compile_model=False, params=params)
    try:
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats(device)
        last_loss = None
        for step in range(args.warmup_steps):
            x, y = batches[step % len(batches)]
            last_loss = train_step(model, optimizer, x, y, loss_fn)
        torch.cuda.synchronize(device)
        sums = [0.0] * 5
        counted = 0
        start = time.perf_counter()
        for step in range(args.timed_steps):
            x, y = batches[step % len(batches)]
            if args.breakdown_timing:
                last_loss, timing = timed_train_step(model, optimizer, x, y, loss_fn, device)
                for i, v in enumerate((timing.zero_grad_ms, timing.forward_ms, timing.loss_ms,
                                       timing.backward_ms, timing.optimizer_ms)):
                    sums[i] += v
                counted += 1
            else:
                last_loss = train_step(model, optimizer, x, y, loss_fn)
        torch.cuda.synchronize(device)
        elapsed = time.perf_counter() - start
        check_recurrences(device)  # raises if a recurrence launch aborted
        ms_per_step = elapsed * 1000.0 / max(args.timed_steps, 1)
        avg = [s / counted for s in sums] if counted else [None] * 5
        steps_per_second = args.timed_steps / elapsed
        return BenchmarkResult(
            **common, ms_per_step=ms_per_step, zero_grad_ms_per_step=avg[0], forward_ms_per_step=avg[1],
            loss_ms_per_step=avg[2], backward_ms_per_step=avg[3], optimizer_ms_per_step=avg[4],
            measured_ms_per_step=sum(avg) if counted else None, steps_per_second=steps_per_second,
            tokens_per_second=steps_per_second * args.batch_size * args.seq_len,
            peak_memory_gb=torch.cuda.max_memory_allocated(device) / (1024.0 ** 3),
            last_loss=float(last_loss.item()) if last_loss is not None else None, status="ok")
    except RuntimeError as e:
        if "out of memory" not in str(e).lower():
            raise
        return BenchmarkResult(**common, ms_per_step=None, zero_grad_ms_per_step=None, forward_ms_per_step=None,
                               loss_ms_per_step=None, backward_ms_per_step=None, optimizer_ms_per_step=None,
                               measured_ms_per_step=None, steps_per_second=None, tokens_per_second=None,
                               peak_memory_gb=None, last_loss=None, status=f"oom: {str(e).splitlines()[0]}")
    finally:
        del optimizer
        del model
        gc.collect()
        torch.cuda.empty_cache()


def write_csv(path: str, results: Iterable[BenchmarkResult]) -> None:
    with open(path, "w", newline="") as f:
        writer = csv.DictWriter(f, fieldnames=CSV_FIELDS)
        writer.writeheader()
        for result in results:
            row = asdict(result)
            writer.writerow({field: row[field] for field in CSV_FIELDS})


def format_result(r: BenchmarkResult) -> str:
    if r.status != "ok":
        return f"{r.cell_type:4s} hidden={r.hidden_size:3d} params={r.params:10d} status={r.status}"
    msg = (f"{r.cell_type:4s} hidden={r.hidden_size:3d} params={r.params:10d} ms/step={r.ms_per_step:9.3f} "
           f"steps/s={r.steps_per_second:8.3f} tokens/s={r.tokens_per_second:12.0f} "
           f"peak_mem={r.peak_memory_gb:6.2f}GB loss={r.last_loss:.6f}")
    if r.measured_ms_per_step is not None:
        msg += (f" breakdown_ms=zero:{r.zero_grad_ms_per_step:.3f},fwd:{r.forward_ms_per_step:.3f},"
                f"loss:{r.loss_ms_per_step:.3f},bwd:{r.backward_ms_per_step:.3f},"
                f"opt:{r.optimizer_ms_per_step:.3f}")
    return msg


def parse_args(argv: Optional[List[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="GRU training-speed benchmark (rnn_kernel_amd).")
    p.add_argument("--hidden-sizes", type=lambda v: [int(x) for x in v.split(",") if x.strip()], default=[256])
    p.add_argument("--batch-size", type=int, default=16)
    p.add_argument("--seq-len", type=int, default=8000)
    p.add_argument("--input-dim", type=int, default=16)
    p.add_argument("--num-layers", type=int, default=4)
    p.add_argument("--sequence-chunk-len", type=int, default=0)
    p.add_argument("--dataset-batches", type=int, default=32)
    p.add_argument("--warmup-steps", type=int, default=3)
    p.add_argument("--timed-steps", type=int, default=10)
    p.add_argument("--lr", type=float, default=3e-4)
    p.add_argument("--seed", type=int, default=42)
    p.add_argument("--device", type=str, default="cuda")
    p.add_argument("--deterministic", action="store_true")
    p.add_argument("--breakdown-timing", action="store_true")
    p.add_argument("--torch-ops", action="store_true",
                   help="use PyTorch's Linear / mse_loss / AdamW around the GRU instead of the HIP ones")
    p.add_argument("--output-csv", type=str, default="")
    return p.parse_args(argv)


def main(argv: Optional[List[str]] = None) -> List[BenchmarkResult]:
    args = parse_args(argv)
    device = torch.device(args.device)
    if device.type != "cuda":
        raise RuntimeError("the GRU path runs on a GPU; --device must be a cuda/hip device")
    torch.manual_seed(args.seed)
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    batches = make_random_batches(args.dataset_batches, args.batch_size, args.seq_len, args.input_dim, device)
    results = []
    for hidden in args.hidden_sizes:
        r = run_case(hidden, batches, args, device)
        print(format_result(r), flush=True)
        results.append(r)
    if args.output_csv:
        write_csv(args.output_csv, results)
    return results


if __name__ == "__main__":
    main()
