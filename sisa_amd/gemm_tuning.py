"""Library GEMM selection for the projection GEMMs around the hot path: the forward and input-gradient products of
the W_cat, W_O, gate/up and down projections, the gate/up weight gradient and the LM head's logits GEMM of the
library arrangement the cross-entropy benchmark times beside its own kernels (the other weight gradients and the
cross-entropy itself run on this library's HIP kernels).

These GEMMs stay on hipBLASLt / rocBLAS through ``torch.mm``/``F.linear``. PyTorch-ROCm's TunableOp can pick, per
GEMM shape and layout, the fastest solution among the libraries' kernels instead of the default heuristic; at the
config-4 training shapes (16,384 rows, K = 768 or 2,744) the heuristic's choices run at 350-680 TFLOP/s and the
measured best ones at 500-1,080. ``enable_tuned_gemms()`` switches TunableOp on in lookup mode with the table shipped
in ``sisa_amd/data/`` (measured on MI355X with this image's ROCm, hipBLASLt and PyTorch; TunableOp ignores a table
whose recorded versions or GPU architecture differ). Shapes not in the table use the default heuristic.

Regenerate the table on the target GPU with ``python -m sisa_amd.gemm_tuning`` (runs the config-4 training step with
tuning on and writes the CSV). TunableOp is process-wide: enabling it affects every GEMM torch issues afterwards.
"""
from __future__ import annotations

import os

import torch

__all__ = ["TABLE", "enable_tuned_gemms", "tune_training_step"]

TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "tunableop_gfx950.csv")


def enable_tuned_gemms(filename: str | None = None) -> bool:
    """Enable TunableOp in lookup mode with ``filename`` (default: the shipped gfx950 table). Returns False (and
    changes nothing) without a GPU, on another architecture, or when the file is missing."""
    path = filename or TABLE
    if not torch.cuda.is_available() or not os.path.exists(path):
        return False
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    if filename is None and arch != "gfx950":
        return False
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(False)
    tun.record_untuned_enable(False)
    tun.set_filename(path)
    return bool(tun.read_file(path))


def tune_training_step(filename: str = TABLE, batch: int = 8, seq_len: int = 2048) -> None:
    """Run the config-4 training step (sisa-152m, bf16 autocast, fused HIP attention, fused linear CE, AdamW) and the
    linear cross-entropy alone at config 3 with TunableOp tuning on, so that every GEMM shape of both is measured; the
    table is written to ``filename``."""
    from sisa_amd import SISAConfig, SISAForCausalLM

    tun = torch.cuda.tunable
    if os.path.exists(filename):
        os.remove(filename)
    tun.enable(True)
    tun.tuning_enable(True)
    tun.set_filename(filename)
    tun.set_max_tuning_duration(100)
    tun.set_max_tuning_iterations(30)
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = SISAConfig.preset("sisa-152m", attn_impl="hip_fused")
    model = SISAForCausalLM(cfg).to(dev)
    opt = torch.optim.AdamW(model.param_groups(3e-4, weight_decay=0.1), betas=(0.9, 0.95), fused=True)
    ids = torch.randint(0, cfg.vocab_size, (batch, seq_len), device=dev)
    for _ in range(2):
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(ids, labels=ids, fused_ce=True).loss
        loss.backward()
        opt.step()
        print(f"tuning step done, loss {float(loss):.4f}, {len(tun.get_results())} GEMM shapes", flush=True)
    # the chunked linear cross-entropy on its own (config 3: 16,384 rows, no label shift)
    from sisa_amd.kernels.linear_ce import linear_cross_entropy

    hidden = torch.randn(batch * seq_len, cfg.d_model, device=dev, requires_grad=True)
    head = (0.02 * torch.randn(cfg.vocab_size, cfg.d_model, device=dev)).requires_grad_(True)
    labels = torch.randint(0, cfg.vocab_size, (batch * seq_len,), device=dev)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ce = linear_cross_entropy(hidden, head, labels)
    ce.backward()
    torch.cuda.synchronize()
    print(f"tuning CE done, {len(tun.get_results())} GEMM shapes", flush=True)
    tun.tuning_enable(False)


if __name__ == "__main__":
    tune_training_step()
    print(f"wrote {TABLE}", flush=True)
