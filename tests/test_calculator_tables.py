"""Per-head reference energies of the calculator (atom_reference * unit of
molfm/data/utils.py:9-289, applied as at model_interface.py:208-223 and
e2former_calculator.py:187-192, 255-260), on the CPU."""
from pathlib import Path

import numpy as np
import pytest

REF_UTILS = Path("/root/reference/src/molfm/data/utils.py")
HARTREE_EV = 27.211386
# Total energies of the isolated ground-state atoms (Hartree; non-relativistic, near the basis-set limit:
# C 3P -37.845, N 4S -54.589, O 3P -75.067, S 3P -398.11).  The molecular-DFT heads' fitted per-element
# references sit within 1% of them for the heavy atoms; H is absorbed differently by the fit (~15-20%).
ATOM_HA = {6: -37.845, 7: -54.589, 8: -75.067, 16: -398.11}


def test_heads_match_by_name_like_the_reference():
    """startswith("svp") / startswith("tzvpd") / == "oc20" / == "omol25" /
    == "oc22" on the lower-cased head name, first match wins; anything else
    gets zeros with unit 1 (the else branch, 128 entries)."""
    from ubio_molfm_amd import calculator as c
    assert c.atom_reference("SVP-enhance")[1] == pytest.approx(0.0433634)
    assert c.atom_reference("tzvpd-small")[1] == pytest.approx(0.0433634)
    assert np.array_equal(c.atom_reference("svp")[0], c.atom_reference("svp-anything")[0])
    assert not np.array_equal(c.atom_reference("svp")[0], c.atom_reference("tzvpd")[0])
    for name, n in (("omol25", 100), ("OMol25", 100), ("oc20", 91), ("oc22", 100)):
        ref, unit = c.atom_reference(name)
        assert unit == 1.0 and len(ref) == n and np.abs(ref).max() > 1.0
    for other in ("omol25-x", "oc20s", "unknown"):
        ref, unit = c.atom_reference(other)
        assert unit == 1.0 and len(ref) == 128 and not ref.any()


def test_molecular_heads_near_isolated_atom_energies():
    """A wrong unit (kcal/mol left unconverted: x23), a table shifted by one
    atomic number (C <-> N differ by 44%) or another head's table in place of
    this one would move these far outside 1%."""
    from ubio_molfm_amd import calculator as c
    for head in ("svp", "tzvpd", "omol25"):
        t = c.head_ref_energy(head)
        for z, ha in ATOM_HA.items():
            ratio = t[z] / (ha * HARTREE_EV)
            assert abs(ratio - 1.0) < 0.01, (head, z, ratio)
        assert -20.0 < t[1] < -13.0, (head, t[1])
        assert abs(t[0]) < 1e-6                                # padding (Z = 0)
        if head == "omol25":                                   # helium (-2.9037 Ha) is in its data
            assert abs(t[2] / (-2.9037 * HARTREE_EV) - 1.0) < 0.05
        else:                                                  # and not in the others'
            assert abs(t[2]) < 1e-3


def test_periodic_heads_per_atom_references():
    """oc20 / oc22 (unit eV): per-atom references of periodic PBE data, the H
    entry near half the PBE energy of H2 (-6.77 eV)."""
    from ubio_molfm_amd import calculator as c
    for head in ("oc20", "oc22"):
        t = c.head_ref_energy(head)
        assert abs(t[1] - (-6.77 / 2)) < 0.1 and t[0] == 0.0 and t[2] == 0.0


@pytest.mark.skipif(not REF_UTILS.exists(), reason="the reference tree is not present on this machine")
def test_shipped_tables_equal_the_reference_source():
    """atom_reference.json equals what make_atom_reference.py reads out of the
    reference file now (the literal arrays and units of every branch)."""
    import json
    from ubio_molfm_amd import make_atom_reference as mk
    shipped = json.loads(mk.OUT.read_text())
    assert mk.extract(str(REF_UTILS)) == shipped
