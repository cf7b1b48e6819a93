"""The committed TunableOp results for the prompt path's library GEMMs (neural_amd/tunableop_mi355x.csv, read by
model.use_tuned_prompt_gemms): validator lines for the PyTorch, HIP, hipBLASLt and rocBLAS versions and the gfx950
target, then one result per bf16 GEMM-with-bias shape of configuration 4's 4,096-token prompt (Q|K|V, o_proj,
router), each an algorithm name and a positive time."""
import csv
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_tuned_prompt_gemms_file():
    from neural_amd.model import TUNED_PROMPT_GEMMS
    assert os.path.abspath(TUNED_PROMPT_GEMMS) == os.path.join(ROOT, "neural_amd", "tunableop_mi355x.csv")
    rows = list(csv.reader(open(TUNED_PROMPT_GEMMS)))
    val = {r[1]: r[2] for r in rows if r[0] == "Validator"}
    assert set(val) >= {"PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "GCN_ARCH_NAME", "ROCBLAS_VERSION"}
    assert val["GCN_ARCH_NAME"].startswith("gfx950")
    res = {r[1]: (r[2], float(r[3])) for r in rows if r[0] != "Validator"}
    # (M, N, K) = (out features, tokens, in features) of Q|K|V, o_proj and the router at T = 4096
    for shape in ("tn_5120_4096_2880_ld_2880_2880_5120", "tn_2880_4096_4096_ld_4096_4096_2880",
                  "tn_128_4096_2880_ld_2880_2880_128"):
        algo, ms = res[shape]
        assert algo and ms > 0.0
    assert all(r[0] == "GemmAndBiasTunableOp_BFloat16_TN" for r in rows if r[0] != "Validator")
