"""The benchmark configurations of the quantized mul_mat hot path.

Shapes follow the FFN projections the reference runs through ggml_mul_mat
(core/src/inference.cpp:1794-1797): W is [N, K] (N output rows, K reduction),
X is [M, K] fp32, Y is [M, N] fp32.
"""
from dataclasses import dataclass

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q4_0 = 2
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
TYPE_Q8_K = 15
TYPE_Q8_0_RS = 108  # row-split Q8_0, the library's load-time repack of Q8_0 rows (dcq_repack_weights)

TYPE_NAMES = {TYPE_Q4_0: "Q4_0", TYPE_Q8_0: "Q8_0", TYPE_Q4_K: "Q4_K", TYPE_Q5_K: "Q5_K", TYPE_Q6_K: "Q6_K",
              TYPE_Q8_K: "Q8_K", TYPE_Q8_0_RS: "Q8_0_RS"}


@dataclass(frozen=True)
class Config:
    index: int
    name: str
    wtype: int
    M: int
    N: int
    K: int
    w_seed: int
    x_seed: int
    w_std: float = 0.02
    outlier_frac: float = 0.0
    outlier_value: float = 20.0
    bound: str = "hbm"

    @property
    def n_outliers(self):
        return int(self.outlier_frac * self.K)


CONFIGS = [
    Config(1, "q8_0_gemv_qwen3_0.6b_ffn_up", TYPE_Q8_0, 1, 3072, 1024, 1001, 2001),
    Config(2, "q4_k_gemv_qwen3_4b_ffn_up", TYPE_Q4_K, 1, 9728, 2560, 1002, 2002),
    Config(3, "q6_k_gemv_qwen3_4b_ffn_down", TYPE_Q6_K, 1, 2560, 9728, 1003, 2003, outlier_frac=0.01),
    Config(4, "q4_k_m64_llama3.2_1b_ffn_up", TYPE_Q4_K, 64, 8192, 2048, 1004, 2004),
    Config(5, "q8_0_prefill_m2048_llama3.2_1b_ffn_up", TYPE_Q8_0, 2048, 8192, 2048, 1005, 2005, bound="mfma"),
]


def by_index(i):
    return CONFIGS[i - 1]
