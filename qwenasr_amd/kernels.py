"""Host mirror of the reference's ``kernels::`` int8 hot-path API on the GPU.

Function names and argument meaning follow crates/qwen-asr/src/kernels/mod.rs;
buffers are :class:`qwenasr_amd.device.DeviceArray` instead of slices, and
every call runs the HIP kernels of libqasr_hip.so on the array's device
(asynchronously on its stream; reading a result back synchronises).
"""
import ctypes as C

from ._lib import QASR_ROUND_HALF_AWAY, P, check, lib


def _h(a):
    return a.dev.h


def quantize_bf16_weights_to_int8(w_bf16, out_dim, in_dim, q, scales, round_mode=QASR_ROUND_HALF_AWAY):
    """kernels/mod.rs:1805 — bf16 [out, in] -> int8 q [out, in] + f32 scales [out]."""
    check(lib().qasr_hip_pack_int8_rows(_h(w_bf16), w_bf16.ptr, out_dim, in_dim, round_mode,
                                        q.ptr, scales.ptr))


def quantize_f32_to_int8(x, q, scale):
    """kernels/mod.rs:1795 — x f32 [k] -> q int8 [k], scale f32 [1] (device)."""
    check(lib().qasr_hip_quantize_act(_h(x), x.ptr, x.shape[-1], q.ptr, scale.ptr))


def linear_int8(y, x, w, ws, bias, in_dim, out_dim):
    """int8_matvec_threaded (kernels/mod.rs:839) with optional bias."""
    check(lib().qasr_hip_linear_int8(_h(x), y.ptr, x.ptr, w.ptr, ws.ptr,
                                     bias.ptr if bias is not None else None, in_dim, out_dim))


def linear_nobias_int8_qkv(q, k, v, x, wq, sq, wk, sk, wv, sv, in_dim, q_dim, kv_dim,
                           norm_w=None, eps=1e-6):
    """kernels/mod.rs:884; with norm_w the rms_norm of decoder.rs:583 is fused in front."""
    if norm_w is None:
        check(lib().qasr_hip_linear_int8_qkv(_h(x), q.ptr, k.ptr, v.ptr, x.ptr, wq.ptr, sq.ptr,
                                             wk.ptr, sk.ptr, wv.ptr, sv.ptr, in_dim, q_dim, kv_dim))
    else:
        check(lib().qasr_hip_rmsnorm_linear_int8_qkv(_h(x), q.ptr, k.ptr, v.ptr, x.ptr, norm_w.ptr,
                                                     eps, wq.ptr, sq.ptr, wk.ptr, sk.ptr, wv.ptr,
                                                     sv.ptr, in_dim, q_dim, kv_dim))


def linear_nobias_int8_swiglu(ffn_out, x, w, ws, in_dim, intermediate, norm_w=None, eps=1e-6):
    """kernels/mod.rs:970 (interleaved gate/up rows); optional fused rms_norm."""
    if norm_w is None:
        check(lib().qasr_hip_linear_int8_swiglu(_h(x), ffn_out.ptr, x.ptr, w.ptr, ws.ptr, in_dim,
                                                intermediate))
    else:
        check(lib().qasr_hip_rmsnorm_linear_int8_swiglu(_h(x), ffn_out.ptr, x.ptr, norm_w.ptr, eps,
                                                        w.ptr, ws.ptr, in_dim, intermediate))


def linear_nobias_int8_addto(y, x, w, ws, in_dim, out_dim):
    """kernels/mod.rs:1030 — y += W x."""
    check(lib().qasr_hip_linear_int8_addto(_h(x), y.ptr, x.ptr, w.ptr, ws.ptr, in_dim, out_dim))


def argmax_matvec_int8(x, w, ws, in_dim, out_dim, out_idx, norm_w=None, eps=1e-6):
    """kernels/mod.rs:1832 — writes the index into out_idx (int32 device [1]) and returns it."""
    if norm_w is None:
        check(lib().qasr_hip_argmax_int8(_h(x), x.ptr, w.ptr, ws.ptr, in_dim, out_dim, out_idx.ptr))
    else:
        check(lib().qasr_hip_rmsnorm_argmax_int8(_h(x), x.ptr, norm_w.ptr, eps, w.ptr, ws.ptr,
                                                 in_dim, out_dim, out_idx.ptr))
    return int(out_idx.numpy().reshape(-1)[0])


def argmax_f32_rows(x, rows, cols, out_idx, ld=None):
    """align.rs:312-321 — per-row argmax of device logits x [rows][ld] into out_idx (int32 device [rows])."""
    check(lib().qasr_hip_argmax_f32_rows(_h(x), x.ptr, cols if ld is None else ld, rows, cols, out_idx.ptr))
    return out_idx.numpy().reshape(-1)[:rows].copy()


def rms_norm(out, x, weight, seq_len, hidden, eps):
    """kernels/mod.rs:1191."""
    check(lib().qasr_hip_rms_norm(_h(x), out.ptr, x.ptr, weight.ptr, seq_len, hidden, eps))


def rms_norm_per_head(x, weight, seq_len, n_heads, head_dim, eps):
    """kernels/mod.rs:1214 (in place)."""
    check(lib().qasr_hip_rms_norm_per_head(_h(x), x.ptr, weight.ptr, seq_len, n_heads, head_dim, eps))


def apply_rope_neox(x, cos_vals, sin_vals, seq, n_heads, head_dim):
    """kernels/mod.rs:1738 (in place)."""
    check(lib().qasr_hip_apply_rope_neox(_h(x), x.ptr, cos_vals.ptr, sin_vals.ptr, seq, n_heads,
                                         head_dim))


def causal_attention(out, q, k_base, v_base, head_stride, seq_q, seq_k, n_heads, n_kv_heads,
                     head_dim, scale, q_offset):
    """kernels/mod.rs:1663 — k_base/v_base are DeviceArrays or raw device pointers."""
    kp = k_base.ptr if hasattr(k_base, "ptr") else k_base
    vp = v_base.ptr if hasattr(v_base, "ptr") else v_base
    check(lib().qasr_hip_causal_attention(_h(q), out.ptr, q.ptr, kp, vp, head_stride, seq_q, seq_k,
                                          n_heads, n_kv_heads, head_dim, scale, q_offset))


def causal_attention_bf16kv(out, q, k_base, v_base, head_stride, seq_k, n_heads, n_kv_heads, head_dim,
                            scale, q_offset):
    """Single-query attention over a bf16 [kv_head][pos][head_dim] cache (config 3)."""
    kp = k_base.ptr if hasattr(k_base, "ptr") else k_base
    vp = v_base.ptr if hasattr(v_base, "ptr") else v_base
    check(lib().qasr_hip_causal_attention_bf16kv(_h(q), out.ptr, q.ptr, kp, vp, head_stride, seq_k, n_heads,
                                                 n_kv_heads, head_dim, scale, q_offset))


def linear(y, x, w_bf16, bias, seq_len, in_dim, out_dim, accumulate=False):
    """linear / linear_accumulate (kernels/mod.rs:550, 591) on bf16-valued weights."""
    check(lib().qasr_hip_linear_bf16w(_h(x), y.ptr, x.ptr, w_bf16.ptr, bias.ptr if bias is not None else None,
                                      seq_len, in_dim, out_dim, 1 if accumulate else 0))


def gemm_w8_bf16(y, a_bf16, w_int8, scales, M, N, K):
    """y[M, N] = (a_bf16 [M, K] . w_int8[N, K]^T) * scales[N] on MFMA."""
    check(lib().qasr_hip_gemm_w8_bf16(_h(a_bf16), y.ptr, a_bf16.ptr, w_int8.ptr, scales.ptr, M, N, K))


def layer_norm(out, x, weight, bias, seq_len, hidden, eps):
    """kernels/mod.rs:1160."""
    check(lib().qasr_hip_layer_norm(_h(x), out.ptr, x.ptr, weight.ptr, bias.ptr, seq_len, hidden, eps))


def bidirectional_attention(out, q, k, v, seq, n_heads, head_dim, scale, window_tokens):
    """kernels/mod.rs:1386 with windows of window_tokens positions."""
    check(lib().qasr_hip_bidirectional_attention(_h(q), out.ptr, q.ptr, k.ptr, v.ptr, seq, n_heads, head_dim,
                                                 scale, window_tokens))
