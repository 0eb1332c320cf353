"""Backbone variants on the CPU (construction only, no GPU calls): attention
types per block ("a+b", e2former.py:792-795,863), the long-range cluster
modules of with_cluster="node*" (e2former.py:887-929) with the reference's
parameter names, and the configurations the reference rejects."""
import pytest
import torch


def _cfg(**over):
    from ubio_molfm_amd import model
    args = model.default_args(num_layers=4)
    args.backbone_config.update(over)
    return args


def test_cluster_modules_and_state_dict_names(pkg):
    from ubio_molfm_amd import model
    from oracle.model import MolfmAtomic as OracleModel
    m = model.MolfmAtomic(_cfg(with_cluster="node_bell", long_range_layers=3, long_cutoff_lower=0.2,
                               long_cutoff_upper=10.0))
    dec = m.decoder.decoder
    assert dec.cluster and len(dec.long_blocks) == 3
    assert all(b.ga.attn_type == "zero-order" and hasattr(b.ga, "proj_zero") for b in dec.long_blocks)
    assert dec.long_envelope() == (1, 0.2)
    assert float(dec.rbf_long.offset[-1]) == 10.0
    assert dec.final_linear.weight.shape == (3, 256, 512)
    om = OracleModel(with_cluster="node_bell", long_range_layers=3, long_cutoff_lower=0.2, long_cutoff_upper=10.0)
    om.load_state_dict(m.state_dict(), strict=True)
    m.load_state_dict(om.state_dict(), strict=True)


def test_block_attention_types(pkg):
    from ubio_molfm_amd import model
    m = model.MolfmAtomic(_cfg(attn_type="so2-first-order+zero-order"))
    types = [b.ga.attn_type for b in m.decoder.decoder.blocks]
    assert types == ["so2-first-order", "so2-first-order", "zero-order", "zero-order"]
    m0 = model.MolfmAtomic(_cfg(attn_type="zero-order"))
    assert m0.decoder.decoder.l3_sequential == [(0, 1), (1, 1), (2, 1)]
    assert not m0.decoder.decoder.cluster


@pytest.mark.parametrize("over, err", [
    (dict(attn_type="zero-order+so2-first-order"), ValueError),
    (dict(with_cluster="edge"), ValueError),
    (dict(attn_type="first-order"), NotImplementedError),
])
def test_rejected_configurations(pkg, over, err):
    from ubio_molfm_amd import model
    with pytest.raises(err):
        model.MolfmAtomic(_cfg(**over))


def test_cluster_polynomial_envelope(pkg):
    from ubio_molfm_amd import model
    dec = model.MolfmAtomic(_cfg(with_cluster="node")).decoder.decoder
    assert dec.cluster and dec.long_envelope() == (0, 0.0)
    assert (dec.long_cutoff_lower, dec.long_cutoff_upper) == (0.1, 12)


@pytest.mark.parametrize("tp", ["QKdot_alpha", "QKdotS_alpha"])
def test_qkdot_variants_state_dict_names(pkg, tp):
    """QKdot_alpha (dot_linear to attn_weight_input_dim, rad_func_m0 with 768
    outputs, fc_m0, an fc_easy of 128) and QKdotS_alpha (sum_vec, dot_linear to
    H // 3 + 1, direction_linear, fc_easy of 256) with the reference's names
    and shapes (e2former.py:143-167): state dicts load both ways, strict."""
    from ubio_molfm_amd import model
    from oracle.model import MolfmAtomic as OracleModel
    m = model.MolfmAtomic(_cfg(tp_type=tp))
    ga = m.decoder.decoder.blocks[0].ga
    if tp == "QKdot_alpha":
        assert ga.dot_linear.weight.shape == (3, 256, 256) and ga.fc_m0.weight.shape == (128, 768)
        assert ga.rad_func_m0.net[6].weight.shape == (768, 128) and ga.fc_easy.net[6].weight.shape == (128, 128)
    else:
        assert ga.dot_linear.weight.shape == (3, 43, 256) and ga.sum_vec.shape == (9, 3)
        assert not ga.sum_vec.requires_grad and ga.fc_easy.net[6].weight.shape == (256, 128)
    om = OracleModel(tp_type=tp)
    om.load_state_dict(m.state_dict(), strict=True)
    m.load_state_dict(om.state_dict(), strict=True)


@pytest.mark.parametrize("tp, form", [("QK_alpha+softplus", "softplus"), ("QK_alpha+sigmoid", "sigmoid"),
                                      ("QKdot_alpha+softplus", "softplus"), ("QKdotS_alpha+sigmoid", "sigmoid"),
                                      ("QK_alpha+sigmoid+softplus", "softplus"), ("QK_alpha", "softmax")])
def test_weight_forms_parsed_like_the_reference(pkg, tp, form):
    """e2former.py:123-124: substring tests on the whole tp_type, softplus
    taking precedence; the parameters are those of the base tp_type, so state
    dicts load both ways."""
    from ubio_molfm_amd import model
    from oracle.model import MolfmAtomic as OracleModel
    m = model.MolfmAtomic(_cfg(tp_type=tp))
    assert all(b.ga.weight_act == form for b in m.decoder.decoder.blocks)
    om = OracleModel(tp_type=tp)
    assert all(b.ga.weight_act == (None if form == "softmax" else form) for b in om.decoder.decoder.blocks)
    om.load_state_dict(m.state_dict(), strict=True)


def test_type_pairs_are_the_products_of_each_graph_type_set(pkg):
    """atom_type_slots: the radial tables' type pairs are the union over graphs
    of each graph's own (a, b) products (edges never leave their graph); every
    pair for a single graph or when the union covers all T^2 (then None)."""
    import torch
    from ubio_molfm_amd import modules
    Z = torch.tensor([1, 6, 1, 8, 8, 16, 1, 6])
    ptr = [0, 3, 6, 8]                      # {1, 6}, {8, 16}, {1, 6}
    tz, (key, pairs), slot = modules.atom_type_slots(Z, ptr)
    assert key == (1, 6, 8, 16) and tz.tolist() == [1, 6, 8, 16] and slot.tolist() == [0, 1, 0, 2, 2, 3, 0, 1]
    assert pairs == ((0, 0), (0, 1), (1, 0), (1, 1), (2, 2), (2, 3), (3, 2), (3, 3))
    assert modules.atom_type_slots(Z)[1][1] is None                          # no graphs: all pairs
    assert modules.atom_type_slots(Z, [0, 8])[1][1] is None                  # one graph
    assert modules.atom_type_slots(torch.tensor([1, 6, 6, 1]), [0, 2, 4])[1][1] is None   # union = all pairs
