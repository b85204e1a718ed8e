"""The Orb-v3 modules called one by one (orb_model.RMSNorm / MLPNorm / Encoder /
AttentionInteractionLayer / EnergyHead ``__call__`` and ``.batch``; reference orb_model.py:107-355)
and their reverse pass (orb_forces.rmsnorm_bw / mlpnorm_bw / attn_layer_bw / energy_bw(_batch) /
backbone_bw(_batch); reference orb_forces.py:67-254) against the fp64 oracle and its autograd,
on the tiny Orb architecture with and without the charge / spin conditioning, edges in an order
that is not sorted by sender."""
import pytest
import torch

from oracle import orb as O
from tt_atom import orb_forces, orb_model
from tt_atom import synthetic as S

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(cond, seed=3):
    cfg = dict(S.CFG_ORB_TINY, has_charge_spin_cond=cond)
    w = S.random_orb_weights(cfg, seed)
    C, H = cfg["latent_dim"], cfg["mlp_hidden_dim"]
    g = torch.Generator().manual_seed(seed)
    N, E = 41, 300
    senders = torch.randint(0, N, (E,), generator=g)
    receivers = (senders + torch.randint(1, N, (E,), generator=g)) % N
    receivers[:40] = 7                                    # a receiver hub
    cut = torch.rand(E, generator=g, dtype=torch.float64) * 0.9 + 0.05
    cond_nodes = torch.randn(N, C, generator=g, dtype=torch.float64) if cond else None
    return cfg, w, C, H, N, E, senders, receivers, cut, cond_nodes, g


def _graph(N, senders, receivers, cut, cond_nodes):
    return orb_model.OrbGraphContext(
        DEV, senders=senders, receivers=receivers, cutoff=cut.float()[:, None], num_nodes=N,
        cond_nodes=None if cond_nodes is None else cond_nodes.float().to(DEV))


def _close(got, ref, tol, what):
    err = (got.detach().cpu().double() - ref).abs().max().item()
    scale = ref.abs().max().item() + 1e-30
    assert err <= tol * scale, f"{what}: max err {err:.3e} vs scale {scale:.3e}"


def _w64(w):
    return {k: torch.as_tensor(v, dtype=torch.float64) for k, v in w.items()}


def test_rmsnorm_and_mlpnorm_modules():
    cfg, w, C, H, N, E, *_ , g = _setup(False)
    w64 = _w64(w)
    # standalone RMSNorm
    rn = orb_model.RMSNorm(w, "_encoder._edge_fn.layer_norm", DEV, C)
    x = torch.randn(57, C, generator=g, dtype=torch.float64)
    xr = x.clone().requires_grad_(True)
    y_ref = O.rmsnorm(xr, w64["_encoder._edge_fn.layer_norm.weight"])
    y = rn(x.float().to(DEV))
    gy = torch.randn(57, C, generator=g, dtype=torch.float64)
    (gx_ref,) = torch.autograd.grad((y_ref * gy).sum(), [xr])
    _close(y, y_ref.detach(), 1e-5, "RMSNorm")
    _close(orb_forces.rmsnorm_bw(rn, gy.float().to(DEV)), gx_ref, 1e-5, "rmsnorm_bw")
    # MLPNorm through the encoder's edge function
    enc = orb_model.Encoder(w, DEV, node_in=cfg["node_embed_size"], edge_in=cfg["edge_embed_size"],
                            latent_dim=C, hidden_dim=H)
    xe = torch.randn(E, cfg["edge_embed_size"], generator=g, dtype=torch.float64)
    xn = torch.randn(N, cfg["node_embed_size"], generator=g, dtype=torch.float64)
    xer = xe.clone().requires_grad_(True)
    ye_ref = O.mlp_norm(xer, w64, "_encoder._edge_fn")
    yn, ye = enc(xn.float().to(DEV), xe.float().to(DEV))
    _close(ye, ye_ref.detach(), 1e-5, "MLPNorm (edge)")
    _close(yn, O.mlp_norm(xn, w64, "_encoder._node_fn"), 1e-5, "MLPNorm (node)")
    ge = torch.randn(E, C, generator=g, dtype=torch.float64)
    (gxe_ref,) = torch.autograd.grad((ye_ref * ge).sum(), [xer])
    _close(orb_forces.mlpnorm_bw(enc.edge_fn, ge.float().to(DEV)), gxe_ref, 2e-5, "mlpnorm_bw")


@pytest.mark.parametrize("cond", [False, True])
def test_attention_layer_module(cond):
    """One layer forward and its adjoints (nodes, edges, cutoff) against the oracle's layer and
    autograd, edges unsorted by sender, a receiver hub, optional conditioning."""
    cfg, w, C, H, N, E, senders, receivers, cut, cond_nodes, g = _setup(cond)
    w64 = _w64(w)
    layer = orb_model.AttentionInteractionLayer(w, "gnn_stacks.0", DEV, latent_dim=C,
                                                hidden_dim=H)
    assert layer.has_cond == cond
    graph = _graph(N, senders, receivers, cut, cond_nodes)
    nodes = torch.randn(N, C, generator=g, dtype=torch.float64)
    edges = torch.randn(E, C, generator=g, dtype=torch.float64)
    nr, er, cr = (t.clone().requires_grad_(True) for t in (nodes, edges, cut))
    n_ref, e_ref = O.attention_layer(nr, er, senders, receivers, cr[:, None], w64, "gnn_stacks.0",
                                     cond_nodes)
    n_out, e_out = layer(nodes.float().to(DEV), edges.float().to(DEV), graph)
    _close(n_out, n_ref.detach(), 2e-5, "layer nodes")
    _close(e_out, e_ref.detach(), 2e-5, "layer edges")
    gn = torch.randn(N, C, generator=g, dtype=torch.float64)
    ge = torch.randn(E, C, generator=g, dtype=torch.float64)
    gn_ref, ge_ref, gc_ref = torch.autograd.grad((n_ref * gn).sum() + (e_ref * ge).sum(),
                                                 [nr, er, cr])
    g_nodes, g_edges, g_cut = orb_forces.attn_layer_bw(layer, graph, gn.float().to(DEV),
                                                       ge.float().to(DEV))
    assert g_cut.shape == (E, 1)
    _close(g_nodes, gn_ref, 5e-5, "attn_layer_bw nodes")
    _close(g_edges, ge_ref, 5e-5, "attn_layer_bw edges")
    _close(g_cut[:, 0], gc_ref, 5e-5, "attn_layer_bw cutoff")


def test_energy_head_and_backbone_bw():
    """EnergyHead (one system and a batch of three) with energy_bw(_batch), and backbone_bw over
    module calls (encoder, both layers, head) against autograd of the oracle's composition."""
    cfg, w, C, H, N, E, senders, receivers, cut, _, g = _setup(False, seed=9)
    w64 = _w64(w)
    eh = orb_model.EnergyHead(w, DEV, latent_dim=C, hidden_dim=H)
    x = torch.randn(N, C, generator=g, dtype=torch.float64)
    xr = x.clone().requires_grad_(True)
    r_ref = O.energy_head(xr, torch.zeros(N, dtype=torch.long), [N], w64)
    raw = eh(x.float().to(DEV))
    assert raw.shape == (1, 1)
    _close(raw[0], r_ref.detach(), 1e-5, "EnergyHead")
    (gx_ref,) = torch.autograd.grad(r_ref.sum(), [xr])
    _close(orb_forces.energy_bw(eh), gx_ref, 1e-5, "energy_bw")
    natoms = [10, 20, N - 30]
    batch = torch.repeat_interleave(torch.arange(3), torch.tensor(natoms))
    seg_mean = torch.zeros(3, N, dtype=torch.float64)
    seg_mean[batch, torch.arange(N)] = 1.0 / torch.tensor(natoms, dtype=torch.float64)[batch]
    xr = x.clone().requires_grad_(True)
    rb_ref = O.energy_head(xr, batch, natoms, w64)
    rb = eh.batch(x.float().to(DEV), seg_mean.float().to(DEV))
    _close(rb[:, 0], rb_ref.detach(), 1e-5, "EnergyHead.batch")
    (gxb_ref,) = torch.autograd.grad(rb_ref.sum(), [xr])
    _close(orb_forces.energy_bw_batch(eh, seg_mean.t().float().to(DEV)), gxb_ref, 1e-5,
           "energy_bw_batch")
    # whole backbone by module calls
    enc = orb_model.Encoder(w, DEV, node_in=cfg["node_embed_size"], edge_in=cfg["edge_embed_size"],
                            latent_dim=C, hidden_dim=H)
    layers = [orb_model.AttentionInteractionLayer(w, f"gnn_stacks.{i}", DEV, latent_dim=C,
                                                  hidden_dim=H)
              for i in range(cfg["num_message_passing_steps"])]
    graph = _graph(N, senders, receivers, cut, None)
    Z = torch.randint(1, 9, (N,), generator=g)
    feat = torch.randn(E, cfg["edge_embed_size"], generator=g, dtype=torch.float64)
    fr, cr = feat.clone().requires_grad_(True), cut.clone().requires_grad_(True)
    e_ref = O.backbone(w64, cfg, Z, fr, cr[:, None], senders, receivers,
                       torch.zeros(N, dtype=torch.long), [N])
    gf_ref, gc_ref = torch.autograd.grad(e_ref.sum(), [fr, cr])
    nodes, edges = enc(O.node_features(w64, Z).float().to(DEV), feat.float().to(DEV))
    for layer in layers:
        nodes, edges = layer(nodes, edges, graph)
    raw = eh(nodes)
    _close(raw[0], e_ref.detach(), 1e-5, "module forward energy")
    g_feat, g_cut = orb_forces.backbone_bw(enc, layers, eh, graph)
    _close(g_feat, gf_ref, 5e-5, "backbone_bw edge features")
    _close(g_cut[:, 0], gc_ref, 5e-5, "backbone_bw cutoff")
