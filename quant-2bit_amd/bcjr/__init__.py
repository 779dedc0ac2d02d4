"""MI355X-native BCJR forward-backward engine for the trellis-coded quantizer.

Python surface mirroring the reference's src/bcjr package; all compute runs in
the gfx950 HIP kernels of libbcjr_hip.so (C ABI in include/bcjr_hip.h).
"""
from .forward_backward import (  # noqa: F401
    BcjrFunction, K_BITS, L_BITS, V_DIM, bcjr_forward_backward, bcjr_forward_backward_fast,
    bcjr_forward_backward_monolithic, bcjr_forward_backward_monolithic_graphed, build_pred_succ_tables,
    reset_mono_graph_cache,
)
from .codes import make_1mad_codebook, make_3inst_codebook, make_hyb_codebook_gpu  # noqa: F401
from .viterbi import (  # noqa: F401
    viterbi_decode_v_batched, viterbi_encode_chunked, viterbi_encode_constrained_v_batched_hip,
    viterbi_encode_tailbiting_v_batched_hip, viterbi_encode_v_batched_cuda, viterbi_encode_v_batched_hip,
)
from .encode import (  # noqa: F401
    viterbi_decode, viterbi_decode_v, viterbi_encode, viterbi_encode_constrained, viterbi_encode_constrained_v,
    viterbi_encode_tailbiting, viterbi_encode_tailbiting_v, viterbi_encode_v, viterbi_encode_v_batched,
)
from .quant import (  # noqa: F401
    bcjr_quantize_tiles, bcjr_quantize_weight, bcjr_quantize_weight_rotated, graphed_bcjr_chunk_forward,
    reset_graph_cache, tile_for_viterbi, untile_from_viterbi,
)
from .rht import (  # noqa: F401
    apply_inverse_rht_batched, apply_inverse_rht_gpu, apply_rht_batched, apply_rht_gpu, hadamard_transform,
    make_sign_vector,
)
from .experts import bcjr_quantize_experts, quantize_moe_experts, ste_quantize_experts  # noqa: F401
from .ste import (  # noqa: F401
    TrellisQuantSTE, TrellisQuantSTE_IP, ptq_residual, quantize_forward_gpu, quantize_forward_gpu_no_rht,
    measure_ptq_residual, quantize_forward_numpy, replay_walks,
)
from .serialize import (  # noqa: F401
    dequant_target, dequant_target_gpu, load_packed, load_quantized, pack_bitstreams, precompute_walk_states,
    save_packed, save_quantized, unpack_bitstreams,
)
from .anneal import bcjr_marginal_entropy, cosine_temperature_schedule, entropy_diagnostic  # noqa: F401
from ._lib import LIB_PATH, load as load_library  # noqa: F401

__version__ = "0.1.0"
