"""The committed TunableOp selections cover the bench's GEMM shapes and are
only read on a GPU (host-side checks, no GPU needed)."""

import csv
import json
from pathlib import Path

from cyclic_flow_attention import gemm_tuning

CONFIG = Path(gemm_tuning.__file__).with_name("configs") / "cyclic_flow_attention_400m.json"


def read_rows():
    with open(gemm_tuning.DEFAULT_FILE, newline="") as f:
        return [r for r in csv.reader(f) if r]


def test_validators_pin_gfx950():
    rows = read_rows()
    validators = {r[1]: r[2] for r in rows if r[0] == "Validator"}
    assert validators["GCN_ARCH_NAME"].startswith("gfx950")
    for key in ("PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION"):
        assert key in validators


def test_selections_cover_the_prefill_projections():
    cfg = json.loads(CONFIG.read_text())
    hidden, vocab = cfg["hidden_size"], cfg["vocab_size"]
    inter = 2 * ((int(hidden * cfg["hidden_ratio"] * 2 / 3) + 255) // 256 * 256)  # gate and up together
    rows = [r for r in read_rows() if r[0] != "Validator"]
    shapes = set()
    for op, sig, solution, ms in rows:
        assert op.startswith(("GemmTunableOp_BFloat16", "GemmAndBiasTunableOp_BFloat16"))
        assert float(ms) > 0
        n, m, k = (int(x) for x in sig.split("_")[1:4])
        shapes.add((n, m, k))
    tokens = 8 * 2048
    for n, k in ((3 * hidden, hidden), (hidden, hidden), (inter, hidden), (hidden, inter // 2), (vocab, hidden)):
        assert (n, tokens, k) in shapes, (n, k)


def test_tuned_gemms_need_a_gpu(tmp_path):
    # without a GPU the selections are not read and nothing is enabled
    assert gemm_tuning.use_tuned_gemms() is False
    assert gemm_tuning.use_tuned_gemms(tmp_path / "missing.csv") is False
