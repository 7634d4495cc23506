"""The ThetaScan token mixer on the hip backend.

Parameters, buffers, names, shapes and initialisation follow the reference
module (src/thetascan/_core/modules/block.py:136-406), so state dicts move
between the two unchanged (including the 40-byte expansion fingerprint and
its strict-load check).  ``forward`` (block.py:573-724) runs in one of two
ways, both on the GPU:

* the fused hot path (``fused.kernel_mixer``) for a depth-1 kernel memory
  with a ReLU^2-ridge or fixed-gain softmax-partition map, raw values, plain
  or key-mass read and the plain temporal sum: three HIP kernels (write,
  scan, read) between the two projection GEMMs;
* the composed path (``engine``) for everything else, where every scan and
  key mass still runs in the HIP kernels.
"""
from __future__ import annotations

import hashlib
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..config import ThetaScanConfig
from ...state import ThetaScanState, config_fingerprint
from ..ops import composed, features, fused, gn, interface, maps, prologue, stream
from ..ops.linear import linear, stack_heads
from ..ops.interface import Accumulator, FadeFast, FadeStale, NullAccumulator, resolve_backend
from .gates import DecayGate, OutGate
from .norms import l2norm
from .rope import apply_rope, rope_cache, rotated_width

_EXPANSION_MAP_DOMAIN = "thetascan-expansion-v1"
_EXPANSION_FINGERPRINT_MAGIC = b"TSXF"
_EXPANSION_FINGERPRINT_SCHEMA_VERSION = 1

FUSED_HEAD_DIMS = (16, 32, 64, 128)
FUSED_FEATURE_WIDTHS = (16, 32, 64, 128, 256)
# widths the chunked feature kernels take: bf16 streams, head widths 32 and 64
WIDE_FEATURE_WIDTHS = (192, 384)
WIDE_HEAD_DIMS = (32, 64)


def _inverse_softplus(value: float) -> float:
    return value + math.log(-math.expm1(-value))


def _row_correlation_penalty(weight: torch.Tensor, eps: float = 1e-8) -> torch.Tensor:
    rows = weight / weight.norm(dim=-1, keepdim=True).clamp_min(eps)
    gram = rows @ rows.t()
    count = gram.shape[0]
    if count < 2:
        return weight.new_zeros(())
    off = gram * (1.0 - torch.eye(count, dtype=gram.dtype, device=gram.device))
    return off.square().sum() / (count * (count - 1))


def _sign_domain(shape, *, key: str, role: str) -> bytes:
    """Versioned SHAKE256 domain of one fixed sign stream (block.py:67-74)."""
    return f"{_EXPANSION_MAP_DOMAIN}\0{key}\0{role}\0{','.join(str(v) for v in shape)}".encode("utf-8")


def _fixed_rademacher(shape, *, key: str, role: str) -> torch.Tensor:
    """Low bit of each SHAKE256 byte -> +-1 (block.py:49-64)."""
    count = math.prod(shape)
    raw = hashlib.shake_256(_sign_domain(shape, key=key, role=role)).digest(count)
    bits = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(torch.int64) & 1
    return (bits.to(torch.float32) * 2.0 - 1.0).reshape(shape)


def _fixed_row_map(shape, *, key: str, role: str, row_norm: float = 1.0, center_rows: bool = True):
    """Deterministic rows of prescribed L2 norm (block.py:117-133)."""
    matrix = _fixed_rademacher(shape, key=key, role=role)
    if center_rows:
        matrix = matrix - matrix.mean(dim=-1, keepdim=True)
    fallback = _fixed_rademacher(shape, key=key, role=f"{role}-fallback")
    norm = matrix.norm(dim=-1, keepdim=True)
    matrix = torch.where(norm > 0.0, matrix, fallback)
    return matrix * (float(row_norm) / matrix.norm(dim=-1, keepdim=True))


def _expansion_fingerprint(*, key: str, effective_hidden: int, feature_expansion: int, depth: int,
                           w1_rows: tuple | None = None):
    """``TSXF || u32 schema || sha256`` identity of the expansion maps (block.py:77-114).

    ``w1_rows`` = (effective, base) rows of the W1 map when they differ from
    the hidden widths: a projected B-spline memory expands its projection rows
    (hidden / basis count), an extension of this build."""
    if feature_expansion <= 1:
        raise ValueError("an expansion fingerprint requires feature_expansion > 1")
    base_hidden = effective_hidden // feature_expansion
    rows_eff, rows_base = w1_rows if w1_rows is not None else (effective_hidden, base_hidden)
    digest = hashlib.sha256()
    digest.update(b"thetascan-expansion-checkpoint\0")
    digest.update(_EXPANSION_MAP_DOMAIN.encode("ascii"))
    for layer in range(depth):
        for desc in (
            _sign_domain((1, rows_eff, rows_base), key=key, role=f"w1-expand-layer-{layer}"),
            _sign_domain((1, base_hidden, effective_hidden), key=key, role=f"w2-expand-layer-{layer}"),
        ):
            digest.update(len(desc).to_bytes(8, "big"))
            digest.update(desc)
    encoded = _EXPANSION_FINGERPRINT_MAGIC + _EXPANSION_FINGERPRINT_SCHEMA_VERSION.to_bytes(4, "big") + digest.digest()
    return torch.tensor(tuple(encoded), dtype=torch.uint8)



class _SplitQKV(torch.autograd.Function):
    """q, k, v [B,H,T,d] views of a stacked [B,T,3,H,d] projection (block.py:594).
    The backward writes the three stream gradients, whatever their strides,
    into one [B,T,3,H,d] gradient in one pass (ts_stack_heads), in the layout
    the projection's backward GEMMs read (autograd's own unbind and permute
    backward stack them head-major and then copy that into this layout)."""

    @staticmethod
    def forward(ctx, proj):
        q, k, v = proj.permute(2, 0, 3, 1, 4).unbind(0)
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        return stack_heads([dq, dk, dv])

class ThetaScan(nn.Module):
    """Drop-in token mixer x[B,T,D] -> y[B,T,D] on MI355X."""

    def __init__(self, cfg: ThetaScanConfig):
        super().__init__()
        self.cfg = cfg
        D, H, d, m, L = cfg.d_model, cfg.n_heads, cfg.head_dim, cfg.mem_hidden, cfg.depth
        if cfg.softmax_gain_mode == "learned_per_head":
            self.kernel_sharpness_raw = nn.Parameter(torch.full((H,), _inverse_softplus(float(cfg.softmax_gain))))
        elif cfg.softmax_gain_mode == "learned_per_feature":
            self.kernel_sharpness_raw = nn.Parameter(torch.full((H, m), _inverse_softplus(float(cfg.softmax_gain))))
        else:
            self.register_parameter("kernel_sharpness_raw", None)
        if cfg.kernel_score_bias:
            self.kernel_score_bias = nn.Parameter(torch.zeros(H, m))
        else:
            self.register_parameter("kernel_score_bias", None)
        if cfg.kernel_relu2_threshold_mode == "learned_per_head":
            self.kernel_relu2_threshold = nn.Parameter(torch.zeros(H))
        else:
            self.register_parameter("kernel_relu2_threshold", None)
        if cfg.kernel_sparsity != "none":
            rho0 = float(cfg.kernel_relative_threshold_init)
            self.kernel_relative_threshold_raw = nn.Parameter(torch.full((H,), math.log(rho0 / (1.0 - rho0))))
        else:
            self.register_parameter("kernel_relative_threshold_raw", None)
        if cfg.kernel_sparsity == "relative_st_blend":
            self.kernel_sparse_blend_raw = nn.Parameter(torch.full((H,), float(cfg.kernel_sparse_blend_init)))
        else:
            self.register_parameter("kernel_sparse_blend_raw", None)
        if cfg.bspline_scale_mode == "learned_per_head":
            self.bspline_scale_raw = nn.Parameter(torch.full((H,), _inverse_softplus(float(cfg.bspline_scale))))
        else:
            self.register_parameter("bspline_scale_raw", None)

        if cfg.key_value_heads is not None:
            G = cfg.key_value_heads
            self.proj_qkv = None
            self.proj_q = nn.Linear(D, H * d, bias=False)
            self.proj_k = nn.Linear(D, G * d, bias=False)
            self.proj_v = nn.Linear(D, G * d, bias=False)
        elif cfg.share_kq:
            self.proj_qkv = None
            self.proj_q1 = nn.Linear(D, d, bias=False)
            self.proj_k1 = nn.Linear(D, d, bias=False)
            self.proj_v = nn.Linear(D, H * d, bias=False)
            self.kq_bias = nn.Parameter(torch.zeros(2, H, d))
        else:
            self.proj_qkv = nn.Linear(D, 3 * H * d, bias=False)
        self.proj_out = nn.Linear(H * d, D, bias=False)

        def w(*shape, fan):
            return nn.Parameter(torch.randn(*shape) / math.sqrt(fan))

        width = m // cfg.feature_expansion
        bspline = cfg.kernel_kind == "projected_bspline"
        # W1 rows: one per feature, or one per projection of a B-spline map
        # (hidden / basis count, block.py:214-222); an expansion widens these
        # rows by feature_expansion (for the B-spline map an extension of this
        # build: 8 trainable projections -> 16 -> 16 x 8 basis = 128 features)
        proj_rows = width // cfg.bspline_basis_count if bspline else width
        rows_eff = m // cfg.bspline_basis_count if bspline else m
        self.W1 = nn.ParameterList([w(H, proj_rows, d, fan=d) for _ in range(L)])
        self.W2 = nn.ParameterList([nn.Parameter(torch.zeros(H, d, width)) for _ in range(L)])
        if cfg.nonlin == "swiglu":
            self.Wg = nn.ParameterList([w(H, m, d, fan=d) for _ in range(L)])
        elif cfg.learn_thresh:
            self.Wg = nn.ParameterList([nn.Parameter(torch.zeros(H, m, 1)) for _ in range(L)])
        elif cfg.value_centers:
            self.Wg = nn.ParameterList([w(1, cfg.value_centers, d, fan=d) for _ in range(L)])
        else:
            self.Wg = None

        self._w1_expansion_buffer_names: tuple = ()
        self._w2_expansion_buffer_names: tuple = ()
        self.register_buffer("_expansion_fingerprint", None)
        if cfg.feature_expansion > 1:
            w1_names, w2_names = [], []
            for layer in range(L):
                w1_name, w2_name = f"_expand_w1_{layer}", f"_expand_w2_{layer}"
                self.register_buffer(w1_name, _fixed_row_map((1, rows_eff, proj_rows), key=cfg.expansion_key,
                                                             role=f"w1-expand-layer-{layer}", center_rows=False),
                                     persistent=False)
                self.register_buffer(w2_name, _fixed_row_map((1, width, m), key=cfg.expansion_key,
                                                             role=f"w2-expand-layer-{layer}", center_rows=False),
                                     persistent=False)
                w1_names.append(w1_name)
                w2_names.append(w2_name)
            self._w1_expansion_buffer_names = tuple(w1_names)
            self._w2_expansion_buffer_names = tuple(w2_names)
            self._expansion_fingerprint = _expansion_fingerprint(
                key=cfg.expansion_key, effective_hidden=m, feature_expansion=cfg.feature_expansion, depth=L,
                w1_rows=(rows_eff, proj_rows))

        self.decay = DecayGate(D, H) if cfg.decay_gate != "off" else None
        self.vmlp_in = self.vmlp_out = None
        if cfg.value_mlp_mult > 0:
            vh = max(1, int(cfg.value_mlp_mult * d))
            self.vmlp_in = nn.Linear(d, vh)
            self.vmlp_out = nn.Linear(vh, d)
            nn.init.zeros_(self.vmlp_out.weight)
            nn.init.zeros_(self.vmlp_out.bias)
        self.ogate = OutGate(D, H, d) if cfg.out_gate else None
        if cfg.read_fade:
            alphas = cfg.resolved_fade_alphas
            if cfg.fade_branches == 1:
                self.fade_alpha = nn.Parameter(torch.full((H,), math.log(alphas[0] / (1.0 - alphas[0]))))
                self.fade_eta = nn.Parameter(torch.zeros(H))
            else:
                raw = [math.log(a / (1.0 - a)) for a in alphas]
                self.fade_alpha = nn.Parameter(torch.tensor(raw).view(-1, 1).expand(-1, H).clone())
                self.fade_eta = nn.Parameter(torch.zeros(cfg.fade_branches, H))
        else:
            self.fade_alpha = None
            self.fade_eta = None
        # The fused path depends only on the (immutable) configuration and on
        # which optional parameters exist, so both are settled here and
        # forward() reads them without writing module state.
        self._views_cfg = self._config_views_eligible()
        self._fused_cfg = self._views_cfg and self._config_fused_eligible()
        self._spec = self._make_feature_spec()
        self.last_path = None

    # ------------------------------------------------------------ checkpoints

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs) -> None:
        """Reject a checkpoint whose expansion fingerprint does not match (block.py:335-406)."""
        fingerprint = self._expansion_fingerprint
        key = prefix + "_expansion_fingerprint"
        if fingerprint is not None and key in state_dict:
            loaded = state_dict[key]
            loaded_bytes = None
            if (torch.is_tensor(loaded) and loaded.dtype == torch.uint8 and loaded.ndim == 1
                    and loaded.numel() == fingerprint.numel()):
                loaded_bytes = bytes(loaded.detach().cpu().tolist())
            expected = bytes(fingerprint.detach().cpu().tolist())
            if loaded_bytes != expected:
                if loaded_bytes is None:
                    reason = "malformed compact fingerprint"
                elif loaded_bytes[:4] != _EXPANSION_FINGERPRINT_MAGIC:
                    reason = "unknown compact fingerprint encoding"
                elif int.from_bytes(loaded_bytes[4:8], "big") != _EXPANSION_FINGERPRINT_SCHEMA_VERSION:
                    reason = (f"unsupported fingerprint schema version {int.from_bytes(loaded_bytes[4:8], 'big')} "
                              f"(expected {_EXPANSION_FINGERPRINT_SCHEMA_VERSION})")
                else:
                    reason = "fingerprint mismatch (different expansion_key, map shapes, or map derivation)"
                error_msgs.append(f"{key}: cannot load random feature expansion: {reason}")
                raise RuntimeError(error_msgs[-1])
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    # ------------------------------------------------------------ controls

    def kernel_sharpness(self):
        if self.kernel_sharpness_raw is None:
            return None
        value = F.softplus(self.kernel_sharpness_raw)
        return value.clamp_min(torch.finfo(value.dtype).tiny)

    def kernel_relative_threshold(self):
        if self.kernel_relative_threshold_raw is None:
            return None
        return torch.sigmoid(self.kernel_relative_threshold_raw)

    def kernel_sparse_blend_alpha(self):
        if self.kernel_sparse_blend_raw is None:
            return None
        bounded = self.kernel_sparse_blend_raw.clamp(0.0, 1.0)
        surrogate = torch.sigmoid(self.kernel_sparse_blend_raw)
        return bounded.detach() + surrogate - surrogate.detach()

    def bspline_scale(self):
        if self.bspline_scale_raw is None:
            return None
        value = F.softplus(self.bspline_scale_raw)
        return value.clamp_min(torch.finfo(value.dtype).tiny)

    def kernel_controls(self) -> dict:
        return {
            "spline_scale": self.bspline_scale(),
            "score_bias": self.kernel_score_bias,
            "relu2_threshold": self.kernel_relu2_threshold,
            "relative_threshold": self.kernel_relative_threshold(),
            "sparse_blend_alpha": self.kernel_sparse_blend_alpha(),
        }

    def key_query_feature_parameters(self):
        seen = set()
        for parameter in self.W1:
            if id(parameter) not in seen:
                seen.add(id(parameter))
                yield parameter
        for name in ("kernel_sharpness_raw", "kernel_score_bias", "kernel_relu2_threshold",
                     "kernel_relative_threshold_raw", "kernel_sparse_blend_raw", "bspline_scale_raw"):
            parameter = getattr(self, name, None)
            if parameter is not None and id(parameter) not in seen:
                seen.add(id(parameter))
                yield parameter

    def fade_blends(self):
        if self.fade_eta is None:
            return None
        return torch.tanh(self.fade_eta) if self.cfg.fade_blend_mode == "tanh" else self.fade_eta

    def ortho_loss(self) -> torch.Tensor:
        """Cosine decorrelation of theta0 rows and heads (block.py:496-544)."""
        cfg = self.cfg
        out = torch.zeros((), device=self.W2[0].device, dtype=self.W2[0].dtype)
        if cfg.ortho_intra == 0.0 and cfg.ortho_inter == 0.0 and cfg.value_mlp_ortho == 0.0:
            return out
        lists = [self.W1, self.W2] + ([] if cfg.learn_thresh else [self.Wg])
        mats = [W for lst in lists if lst is not None for W in lst]
        if cfg.ortho_intra:
            eligible = [W for W in mats if W.shape[-2] > 1]
            acc = 0.0
            for W in eligible:
                Wn = W / W.norm(dim=-1, keepdim=True).clamp_min(cfg.eps)
                G = Wn @ Wn.transpose(-1, -2)
                r = G.shape[-1]
                off = G * (1.0 - torch.eye(r, device=G.device, dtype=G.dtype))
                acc = acc + off.square().sum() / (G.shape[0] * r * (r - 1))
            if eligible:
                out = out + cfg.ortho_intra * acc / len(eligible)
        if cfg.ortho_inter and cfg.n_heads > 1:
            eligible = [W for W in mats if W.shape[0] > 1]
            acc = 0.0
            for W in eligible:
                V = W.flatten(1)
                Vn = V / V.norm(dim=-1, keepdim=True).clamp_min(cfg.eps)
                Gh = Vn @ Vn.t()
                Hh = Gh.shape[0]
                off = Gh * (1.0 - torch.eye(Hh, device=Gh.device, dtype=Gh.dtype))
                acc = acc + off.square().sum() / (Hh * (Hh - 1))
            if eligible:
                out = out + cfg.ortho_inter * acc / len(eligible)
        if cfg.value_mlp_ortho and self.vmlp_in is not None:
            out = out + cfg.value_mlp_ortho * (_row_correlation_penalty(self.vmlp_in.weight, cfg.eps)
                                               + _row_correlation_penalty(self.vmlp_out.weight, cfg.eps)) / 2.0
        return out

    def _weights(self):
        """Effective (expanded) memory weights per depth level (block.py:546-567)."""
        out = []
        for l in range(self.cfg.depth):
            W1, W2 = self.W1[l], self.W2[l]
            if self.cfg.feature_expansion > 1:
                W1 = torch.matmul(getattr(self, self._w1_expansion_buffer_names[l]).to(W1.dtype), W1)
                W2 = torch.matmul(W2, getattr(self, self._w2_expansion_buffer_names[l]).to(W2.dtype))
            out.append((W1, W2, self.Wg[l] if self.Wg is not None else None))
        return out

    # ------------------------------------------------------------ forward

    def fused_eligible(self, x: torch.Tensor) -> bool:
        """Whether the HIP feature kernels carry this configuration and input
        (the one-call sum path or the multi-view path)."""
        if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float32):
            return False
        if self.cfg.mem_hidden in WIDE_FEATURE_WIDTHS and x.dtype != torch.bfloat16:
            return False
        return self._views_cfg

    def _config_views_eligible(self) -> bool:
        """The kernel memory that ts_feature_fwd / ts_feature_bwd compute: depth
        1, one write, L2-normed keys and queries, the ReLU^2 ridge (with or
        without the per-head threshold) or the fixed-gain dense softmax
        partition, widths the kernels take, and a plain or key-mass read;
        any projection layout, value MLP and temporal mode."""
        cfg = self.cfg
        if cfg.write_rule != "kernel" or cfg.depth != 1 or cfg.write_iters != 1 or cfg.value_centers:
            return False
        if not cfg.qk_norm:
            return False
        if cfg.read_norm and cfg.read_norm_mode != "key_mass":
            return False
        wide = cfg.mem_hidden in WIDE_FEATURE_WIDTHS and cfg.head_dim in WIDE_HEAD_DIMS
        if cfg.head_dim not in FUSED_HEAD_DIMS or (cfg.mem_hidden not in FUSED_FEATURE_WIDTHS and not wide):
            return False
        rot_in = rotated_width(cfg.head_dim, cfg.rope, cfg.rope_frac) if cfg.rope_placement == "input" else 0
        rot_feat = rotated_width(cfg.mem_hidden, cfg.rope, cfg.rope_frac) if cfg.rope_placement == "feature" else 0
        if rot_in % 4 or rot_feat % 4:
            return False
        if cfg.kernel_kind == "relu2_ridge":
            return self.kernel_score_bias is None
        if cfg.kernel_kind == "softmax_partition":
            return (cfg.softmax_gain_mode == "fixed" and cfg.kernel_sparsity == "none"
                    and self.kernel_score_bias is None)
        return False

    def _config_fused_eligible(self) -> bool:
        """The one-call sum path (ts_memory_fwd / ts_memory_bwd between the
        stacked projection and the output projection): a views-eligible memory
        with the plain sum and the stacked qkv projection, at a feature width
        with in-kernel weight-gradient partials."""
        cfg = self.cfg
        return not (cfg.read_fade or cfg.accumulation != "sum" or cfg.share_kq or cfg.key_value_heads is not None
                    or cfg.value_mlp_mult > 0 or cfg.mem_hidden in WIDE_FEATURE_WIDTHS)

    def _make_feature_spec(self):
        cfg = self.cfg
        d, m = cfg.head_dim, cfg.mem_hidden
        in_rot = rotated_width(d, cfg.rope, cfg.rope_frac) if cfg.rope_placement == "input" else 0
        feat_rot = rotated_width(m, cfg.rope, cfg.rope_frac) if cfg.rope_placement == "feature" else 0
        kind = fused._lib.FEAT_RELU2 if cfg.kernel_kind == "relu2_ridge" else fused._lib.FEAT_SOFTMAX
        return fused.FeatureSpec(kind, m, cfg.softmax_gain, in_rot, feat_rot, cfg.rope_base,
                                 1.0 / math.sqrt(cfg.depth), cfg.eps)

    def _forward_fused(self, x: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        H = cfg.n_heads
        spec = self._spec
        (W1, W2, _), = self._weights()
        gate = self.ogate is not None
        return fused.kernel_mixer(x, self.proj_qkv.weight, self.ogate.g.lin.weight if gate else None,
                                  self.ogate.g.lin.bias if gate else None, W1, W2, self.kernel_relu2_threshold,
                                  self.proj_out.weight, spec, cfg.read_norm, H)

    def _fingerprint(self) -> str:
        """config_fingerprint(self.cfg), recomputed only when a field changes
        (the configuration's fields are flat values: a shallow snapshot sees
        every change)."""
        snap = tuple(self.cfg.__dict__.items())
        memo = self.__dict__.get("_fingerprint_memo")
        if memo is None or memo[0] is not self.cfg or memo[1] != snap:
            memo = (self.cfg, snap, config_fingerprint(self.cfg))
            self.__dict__["_fingerprint_memo"] = memo
        return memo[2]

    def initial_state(self) -> ThetaScanState:
        """The state of a sequence with no tokens yet (streaming continuation)."""
        return ThetaScanState(fingerprint=self._fingerprint())

    def forward(self, x: torch.Tensor, state: ThetaScanState | None = None):
        """``y`` for ``x`` [B,T,D]; with ``state``, the sequence continues from
        it and ``(y, new_state)`` is returned (no autograd)."""
        cfg = self.cfg
        backend = resolve_backend(cfg.backend, cfg.decay_gate, cfg.accumulation, device=x.device,
                                  require_scalar_decay=cfg.read_fade)
        if not x.is_cuda:
            raise RuntimeError("the hip backend runs on the GPU only (no CPU fallback)")
        if state is not None:
            return self._forward_carried(x, state, backend)
        fused_path = self.fused_eligible(x)
        if not torch.compiler.is_compiling():
            # a record for eager callers; a traced forward writes no module state
            self.last_path = "fused" if fused_path else "composed"
        if fused_path:
            return self._forward_fused(x) if self._fused_cfg else self._forward_views(x, backend)
        return self._forward_composed(x, backend)

    def _forward_carried(self, x: torch.Tensor, state: ThetaScanState, backend: str):
        """One call of a continued sequence: every scan and decayed prefix of
        the forward starts from the state the previous call left (the
        one-call sum path keeps no state, so the multi-view path serves it)."""
        if state.fingerprint != self._fingerprint():
            raise ValueError("this state belongs to a mixer of another configuration")
        B = x.shape[0]
        if state.carries and state.batch != B:
            raise ValueError(f"the state holds {state.batch} sequences; the input has {B}")
        for t in state._tensors():
            if t.device != x.device:
                raise ValueError(f"the state lives on {t.device}; the input on {x.device} (use state.to)")
        if x.shape[1] == 0:
            # no tokens: the memory is unchanged
            with stream.carrying(stream.Carry()):
                return x.new_empty(B, 0, self.proj_out.weight.shape[0]), state
        carry = stream.Carry(state.carries, state.position)
        with stream.carrying(carry):
            if self.fused_eligible(x):
                self.last_path = "fused"
                y = self._forward_views(x, backend)
            else:
                self.last_path = "composed"
                y = self._forward_composed(x, backend)
        if state.carries and len(carry.out) != len(state.carries):
            raise RuntimeError("the state does not match this forward's scans")
        return y, ThetaScanState(fingerprint=state.fingerprint, position=state.position + x.shape[1], batch=B,
                                 carries=tuple(carry.out))

    def _project(self, x):
        cfg = self.cfg
        B, T, _ = x.shape
        H, d = cfg.n_heads, cfg.head_dim
        if cfg.key_value_heads is not None:
            G = cfg.key_value_heads
            q = linear(x, self.proj_q.weight).view(B, T, H, d).transpose(1, 2)
            k = linear(x, self.proj_k.weight).view(B, T, G, d).transpose(1, 2)
            v = linear(x, self.proj_v.weight).view(B, T, G, d).transpose(1, 2)
            return q, k.repeat_interleave(H // G, dim=1), v.repeat_interleave(H // G, dim=1)
        if cfg.share_kq:
            kqb = self.kq_bias.to(dtype=x.dtype)
            q = linear(x, self.proj_q1.weight).unsqueeze(1) + kqb[0][None, :, None, :]
            k = linear(x, self.proj_k1.weight).unsqueeze(1) + kqb[1][None, :, None, :]
            v = linear(x, self.proj_v.weight).view(B, T, H, d).transpose(1, 2)
            return q, k, v
        return _SplitQKV.apply(linear(x, self.proj_qkv.weight).view(B, T, 3, H, d))

    def _forward_composed(self, x: torch.Tensor, backend: str = "hip") -> torch.Tensor:
        cfg = self.cfg
        B, T, _ = x.shape
        H, d = cfg.n_heads, cfg.head_dim
        q, k, v = self._project(x)
        rot_in = rotated_width(d, cfg.rope, cfg.rope_frac) if cfg.rope_placement == "input" else 0
        qn = kn = None
        if cfg.qk_norm:
            # input RoPE + L2 norm in one HIP kernel per stream (strided views in)
            qn = prologue.qk_norm(q, rot_in, cfg.rope_base, cfg.eps)
            kn = prologue.qk_norm(k, rot_in, cfg.rope_base, cfg.eps) if qn is not None else None
        if qn is not None and kn is not None:
            q, k = qn, kn
        else:
            if cfg.rope_placement == "input":
                q = apply_rope(q, cfg.rope, cfg.rope_frac, cfg.rope_base)
                k = apply_rope(k, cfg.rope, cfg.rope_frac, cfg.rope_base)
            if cfg.qk_norm:
                q, k = l2norm(q, cfg.eps), l2norm(k, cfg.eps)
        v_w = v
        if self.vmlp_in is not None:
            v_w = v_w + self.vmlp_out(F.silu(self.vmlp_in(v_w)))
        hrot = None
        if cfg.rope_placement == "feature" and cfg.rope != "none":
            rot = rotated_width(cfg.mem_hidden, cfg.rope, cfg.rope_frac)
            if rot:
                hcos, hsin = rope_cache(T, rot, cfg.rope_base, x.device, x.dtype)
                hrot = (hcos, hsin, rot)
        views, etas = self._temporal_views(x, backend)
        weights = self._weights()
        sharp = self.kernel_sharpness()
        controls = self.kernel_controls()
        gate = self._read_gate(x, views)
        reads = composed.memory_forward(weights, cfg, k, v_w, q, tuple(views), hrot=hrot, gain=sharp,
                                        controls=controls, out_gate=gate)
        if gate is not None and gate.applied:
            # the read epilogue applied the output gate and wrote its output
            # token-major: the projection reads it as [B,T,H*d] in place
            return linear(reads[0].transpose(1, 2).reshape(B, T, H * d), self.proj_out.weight)
        return self._blend_and_project(x, reads, etas)

    def _read_gate(self, x: torch.Tensor, views):
        """The output gate (block.py:721-722) as a request that the HIP read
        epilogue of a single view may apply (composed.GateRequest), or None
        where the gate stays a product after the read (banks: after the
        blend)."""
        cfg = self.cfg
        if self.ogate is None or cfg.read_fade or len(views) != 1 or not x.is_cuda:
            return None
        lin = self.ogate.g.lin
        return composed.GateRequest(x, lin.weight, lin.bias, cfg.n_heads, cfg.head_dim)

    def _temporal_views(self, x: torch.Tensor, backend: str):
        """The memory's temporal views (interface.py:198-327): the accumulator
        (plain sum or the ema stream) and, for a bank, one fast or stale view
        per recency branch (block.py:647-681), with the branches' blends."""
        cfg = self.cfg
        B, T, _ = x.shape
        H = cfg.n_heads
        decay_d = decay_m = None
        if self.decay is not None:
            decay_d, decay_m = self.decay(x)
        acc = Accumulator(backend, decay_d=decay_d, decay_m=decay_m, eps=cfg.eps, chunk=cfg.scan_chunk)
        views = [acc]
        etas = []
        if cfg.read_fade:
            alpha_raw = self.fade_alpha
            eta = self.fade_blends()
            if alpha_raw.ndim == 1:
                alpha_raw, eta = alpha_raw.unsqueeze(0), eta.unsqueeze(0)
            for branch in range(cfg.fade_branches):
                log_alpha = (-F.softplus(-alpha_raw[branch])).to(dtype=x.dtype)
                la_s = log_alpha.view(1, H, 1, 1).expand(B, H, T, 1)
                fast = Accumulator(backend, decay_d=la_s, decay_m=la_s, eps=cfg.eps, chunk=cfg.scan_chunk,
                                   static_log_alpha=log_alpha)
                if cfg.read_fade_mode == "fast":
                    views.append(FadeFast(fast, log_alpha, chunk=cfg.scan_chunk))
                else:
                    views.append(FadeStale(acc, fast, log_alpha, cfg.scan_chunk))
                etas.append(eta[branch].view(1, -1, 1, 1))
            if cfg.read_fade_mode == "stale":
                views.append(NullAccumulator())
        return views, etas

    def _blend_and_project(self, x: torch.Tensor, reads, etas) -> torch.Tensor:
        """Bank blend (block.py:683-717), output gate and projection (block.py:721-724)."""
        cfg = self.cfg
        B, T, _ = x.shape
        y = reads[0]
        if cfg.read_fade:
            coef = maps.fast_coefficients(etas) if cfg.read_fade_mode == "fast" else maps.stale_coefficients(etas)
            if (self.ogate is not None and not torch.is_grad_enabled() and x.is_cuda
                    and all(r.dtype == x.dtype for r in reads) and self.ogate.g.lin.weight.dtype == x.dtype):
                # inference: the output gate in the blend's epilogue (one
                # launch, no gate or transposing copy of the blended read)
                lin = self.ogate.g.lin
                pre = linear(x, lin.weight).view(B, T, cfg.n_heads, cfg.head_dim).transpose(1, 2)
                y = maps.bank_blend_gated(reads, coef, pre, lin.bias)
                return linear(y.transpose(1, 2).reshape(B, T, cfg.n_heads * cfg.head_dim), self.proj_out.weight)
            y = maps.bank_blend(reads, coef)
        if self.ogate is not None:
            y = y * self.ogate(x)
        y = y.transpose(1, 2).reshape(B, T, cfg.n_heads * cfg.head_dim)
        return linear(y, self.proj_out.weight)

    def _forward_views(self, x: torch.Tensor, backend: str = "hip") -> torch.Tensor:
        """The kernel memory on the HIP feature kernels for any projection
        layout and temporal mode: the raw key and query streams go through
        ts_feature_fwd (input RoPE, L2 norm, W1, RMSNorm, threshold, feature
        map, feature RoPE, and the query's residual xn + s W2 h), every view
        is scanned by the multi-view scan and read by ts_read_fwd
        (engine.py:345-544 for depth 1, write_iters 1)."""
        cfg = self.cfg
        q, k, v = self._project(x)
        v_w = v
        if self.vmlp_in is not None:
            v_w = v_w + self.vmlp_out(F.silu(self.vmlp_in(v_w)))
        (W1, W2, _), = self._weights()
        tau = self.kernel_relu2_threshold
        phi_k, _ = features.kernel_features(k, W1, None, tau, self._spec, False)
        phi_q, resid = features.kernel_features(q, W1, W2, tau, self._spec, True)
        views, etas = self._temporal_views(x, backend)
        s = 1.0 / math.sqrt(cfg.depth)
        if cfg.read_norm:
            pairs = interface.scan_views_mass(tuple(views), phi_q, phi_k, v_w, "m")
        else:
            pairs = [(num, None) for num in interface.scan_views(tuple(views), phi_q, phi_k, v_w, "m")]
        reads = [gn.normalized_read(num, mass, resid, s=s, eps=cfg.eps) for num, mass in pairs]
        return self._blend_and_project(x, reads, etas)
