"""The two-layer MACE model evaluated by the three-pass path: architecture, parameters and derived tables.

The reference evaluates a mace-torch 0.3.15 ``ScaleShiftMACE`` (MACE-MPA-0 medium or the same architecture)
whose blocks it reaches through ``model.interactions[k]``, ``model.products[k]``, ``model.readouts[k]``
(receiver_chunk_mace.py:230-256, fast_layers.py:168-222).  mace-torch is not part of this build, so the
architecture is restated here from its definition (block types asserted at fast_layers.py:117-119):

  node_feats   = onehot @ W_emb / sqrt(n_el)                                    (89x0e -> 128x0e)
  edge         : v = x_recv - x_send, r = |v|, Y = SH_l<=3(v/r) (16 comps), B = Bessel_8(r), f = cutoff_p5(r)
  layer k      : X      = linear_up(node_feats)
                 W_e    = MLP[8,64,64,64,nW*128](B) * f          (radial weights per TP path and channel)
                 d_e    = tanh((B @ w_dens / sqrt(8))^2) * f     (edge density)
                 A_i    = sum_{e -> i} TP_uvu(W_e, X[send_e], Y_e)   -> mid irreps
                 M_i    = linear(A_i) / (sum_{e -> i} d_e + 1)
                 layer 1: M_i = skip_tp(M_i, species_i) ; sc = None
                 layer 2: sc_i = skip_tp(node_feats_i, species_i)     (0e part -> 128x0e)
                 h_i    = linear(SymmetricContraction_corr3(M_i, species_i)) (+ sc_i)
  readouts     : R1(h1) = h1[0e] @ w / sqrt(128) ;  R2(h2) = silu_n(h2 @ W1 / sqrt(128)) @ w2 / sqrt(16)
  energy       : E_i = e0[Z_i] + shift + scale * (R1(h1_i) + R2(h2_i))

Normalisations follow e3nn's conventions (weights ~ N(0, 1); Linear: 1/sqrt(fan_in) summed over the paths
into one output; FullyConnectedNet: h <- silu_n(h @ W / sqrt(fan_in)) with silu_n = normalize2mom(silu);
FullyConnectedTensorProduct with a one-hot: 1/sqrt(mul_in * n_el)).  Choices the benchmark specification leaves
open and this build fixes: no Agnesi distance transform, no ZBL pair repulsion, the cutoff multiplies the
radial-MLP output and the density (mace's ``cutoff is not None`` branch, fast_layers.py:190-192), silu_n's
constant by quadrature.
Features are stored "ir_mul" (component-major, channel-minor), as in the reference (make_threepass_model.py:42).
"""

import torch

from . import o3

# normalize2mom(silu): 1 / sqrt(E_{z ~ N(0,1)} silu(z)^2), by adaptive quadrature (e3nn estimates the same
# constant by Monte-Carlo)
SILU_NORM = 1.6765324703310913

LAYER1_IN = [0]            # node feats of layer 1: 128x0e
HIDDEN = [0, 1]            # h1: 128x0e + 128x1o
TARGET = [0, 1, 2, 3]      # interaction irreps: 128x(0e+1o+2e+3o)
HIDDEN_OUT2 = [0]          # h2: 128x0e


class MaceSpec:
    """Architecture of the random-init "MPA-0-medium" model of the benchmark configurations."""

    def __init__(self, num_elements=89, C=128, r_max=6.0, num_bessel=8, p_cutoff=5, radial_mlp=(64, 64, 64),
                 correlation=3, mlp_irreps=16, scale=1.0, shift=0.0):
        self.num_elements = int(num_elements)
        self.atomic_numbers = list(range(1, self.num_elements + 1))
        self.C = int(C)
        self.r_max = float(r_max)
        self.num_bessel = int(num_bessel)
        self.p_cutoff = int(p_cutoff)
        self.radial_mlp = [int(h) for h in radial_mlp]
        self.correlation = int(correlation)
        self.mlp_irreps = int(mlp_irreps)
        self.scale = float(scale)
        self.shift = float(shift)

    def as_dict(self):
        return dict(self.__dict__)


class Tables:
    """Architecture-derived coupling tables (pure data; deterministic)."""

    def __init__(self, spec):
        self.tp1 = o3.tp_table(LAYER1_IN, 3, TARGET)          # nX=1, nW=4,  nO=16, 16 terms
        self.tp2 = o3.tp_table(HIDDEN, 3, TARGET)             # nX=4, nW=10, nO=40, 86 terms
        self.sc1 = {L: o3.symmetric_contraction_paths(TARGET, L, spec.correlation) for L in HIDDEN}
        self.sc2 = {L: o3.symmetric_contraction_paths(TARGET, L, spec.correlation) for L in HIDDEN_OUT2}
        # lin2: output l <- every mid segment of layer 2 with irrep l (in mid order)
        self.lin2_src = {l: [w for w, lw in enumerate(self.tp2["mid_ls"]) if lw == l] for l in TARGET}


def _pname(*parts):
    return "_".join(str(p) for p in parts)


class MaceModel(torch.nn.Module):
    """Parameters of the two-layer model in one flat ParameterDict (fp32 values).

    Parameter names (shapes with C=128, n_el=89, B=8):
      emb [n_el, C]
      i0_up [C, C] ; i0_r0 [B, 64], i0_r1 [64, 64], i0_r2 [64, 64], i0_r3 [64, 4C] ; i0_dens [B, 1]
      i0_lin [4, C, C] (l = 0..3) ; i0_skip [4, C, n_el, C]
      p0_w_L{L}_nu{nu} [n_el, K, C] for L in (0, 1), nu in 1..3 ; p0_lin [2, C, C] ; r0 [C]
      i1_skip [C, n_el, C] ; i1_up [2, C, C] (l = 0, 1)
      i1_r0.. i1_r3 [64, 10C] ; i1_dens [B, 1] ; i1_lin_l{l} [n_src(l), C, C]
      p1_w_L0_nu{nu} [n_el, K, C] ; p1_lin [1, C, C] ; r1_w1 [C, 16], r1_w2 [16]
      e0 [n_el] (buffer)
    """

    def __init__(self, spec=None, seed=0, dtype=torch.float32):
        super().__init__()
        spec = spec or MaceSpec()
        self.spec = spec
        self.tables = Tables(spec)
        C, ne, nb = spec.C, spec.num_elements, spec.num_bessel
        g = torch.Generator().manual_seed(int(seed))

        def rn(*shape, scale=1.0):
            return torch.nn.Parameter(torch.randn(*shape, generator=g, dtype=torch.float64) * scale,
                                      requires_grad=False)

        p = {}
        p["emb"] = rn(ne, C)
        hs = spec.radial_mlp
        for k, (tab, up_ls) in enumerate(((self.tables.tp1, LAYER1_IN), (self.tables.tp2, HIDDEN))):
            if k == 1:
                p["i1_skip"] = rn(C, ne, C)
            p[_pname(f"i{k}", "up")] = rn(len(up_ls), C, C)
            dims = [nb] + hs + [tab["nW"] * C]
            for j in range(len(dims) - 1):
                p[_pname(f"i{k}", f"r{j}")] = rn(dims[j], dims[j + 1])
            p[_pname(f"i{k}", "dens")] = rn(nb, 1)
            if k == 0:
                p["i0_lin"] = rn(len(TARGET), C, C)
                p["i0_skip"] = rn(len(TARGET), C, ne, C)
            else:
                for l in TARGET:
                    p[_pname("i1_lin", f"l{l}")] = rn(len(self.tables.lin2_src[l]), C, C)
            sc = self.tables.sc1 if k == 0 else self.tables.sc2
            for L in sorted(sc):
                for nu in sorted(sc[L]):
                    K = len(sc[L][nu])
                    p[_pname(f"p{k}", "w", f"L{L}", f"nu{nu}")] = rn(ne, K, C, scale=1.0 / K)
            p[_pname(f"p{k}", "lin")] = rn(len(sc), C, C)
            if k == 0:
                p["r0"] = rn(C)
            else:
                p["r1_w1"] = rn(C, spec.mlp_irreps)
                p["r1_w2"] = rn(spec.mlp_irreps)
        # the canonical weights are fp32 numbers (the reference's production model is fp32): the fp64 oracle and the
        # fp32 kernels then start from identical parameter values
        for v in p.values():
            v.data = v.data.float().double()
        self.p = torch.nn.ParameterDict(p)
        self.register_buffer("e0", torch.zeros(ne, dtype=torch.float64))
        # radial networks per ordered element pair: {(sender column, receiver column): {block k: [r0, .., r3]}}
        # for models whose radial weights depend on the species pair (MACE-MPA-0's species-pair distance transform
        # makes W(r) a different function for every ordered pair); pairs not listed use i{k}_r*.  None: one
        # network per block for all pairs (this architecture).  The kernels then read one spline table per
        # distinct network (FastLayers).
        self.pair_radial = None
        self.to(dtype)

    # -- attributes the ML-IAP wrapper reads from a mace model
    @property
    def atomic_numbers(self):
        return torch.tensor(self.spec.atomic_numbers)

    @property
    def r_max(self):
        return torch.tensor(self.spec.r_max)

    def forward(self, *a, **k):   # pragma: no cover - the model is evaluated by the three-pass path only
        raise RuntimeError("MaceModel holds parameters; evaluate it with ThreePassMLIAP or ReceiverChunkMACE")


def load_weights(model, path):
    """Loads a state_dict (safetensors, or a weights-only torch file) into the model, every parameter required."""
    if path.endswith(".safetensors"):
        from safetensors.torch import load_file
        sd = load_file(path)
    else:
        sd = torch.load(path, map_location="cpu", weights_only=True)
    model.load_state_dict(sd, strict=True)
    return model


def from_arg(arg):
    """The --model option of the command-line entry points: "seed:N" gives the random-init architecture with seed
    N; anything else names a weights file for it (load_weights)."""
    if arg.startswith("seed:"):
        return MaceModel(seed=int(arg[5:]))
    return load_weights(MaceModel(seed=0), arg)
