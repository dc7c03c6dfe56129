"""Structure input of the command-line entry points (CPU): the extended-XYZ, LAMMPS-data and npz readers against
the arrays they were written from, periodic replicas, the shared structure options, the element tables, and the
command lines' argument handling."""
import numpy as np
import pytest

from mace_onegpu import systems


def _water():
    return systems.water_box(64, seed=2)


def test_extxyz_round_trip(tmp_path):
    pos, box, Z = _water()
    f = tmp_path / "w.extxyz"
    r = lambda v: repr(float(v))                                     # shortest round-trip decimal
    lines = [str(len(pos)), f'Lattice="{r(box[0])} 0 0 0 {r(box[1])} 0 0 0 {r(box[2])}" Properties=species:S:1:pos:R:3']
    lines += [f"{systems.SYMBOLS[z - 1]} {r(x)} {r(y)} {r(w)}" for z, (x, y, w) in zip(Z, pos)]
    f.write_text("\n".join(lines) + "\n")
    p2, b2, z2 = systems.read_structure(str(f))
    assert np.array_equal(p2, pos) and np.array_equal(b2, box) and np.array_equal(z2, Z)


def test_lammps_data_types_ids_and_origin(tmp_path):
    """Atom types map to Z through the type list (1 = O, 2 = H by default), rows come back in id order, and a box
    that starts at xlo != 0 is shifted to [0, L)."""
    pos, box, Z = _water()
    lo = np.array([-5.0, 2.5, 0.0])
    order = np.random.default_rng(0).permutation(len(pos))          # rows written in shuffled id order
    r = lambda v: repr(float(v))
    rows = [f"{i + 1} {1 if Z[i] == 8 else 2} {r(pos[i, 0] + lo[0])} {r(pos[i, 1] + lo[1])} {r(pos[i, 2] + lo[2])} 0 0 0"
            for i in order]
    text = ["LAMMPS data file", "", f"{len(pos)} atoms", "2 atom types", ""]
    text += [f"{r(lo[d])} {r(lo[d] + box[d])} {c}lo {c}hi" for d, c in enumerate("xyz")]
    text += ["", "Masses", "", "1 15.999", "2 1.008", "", "Atoms # atomic", ""] + rows
    f = tmp_path / "w.data"
    f.write_text("\n".join(text) + "\n")
    p2, b2, z2 = systems.read_structure(str(f))
    assert np.array_equal(z2, Z)
    np.testing.assert_allclose(p2, pos, atol=1e-12)
    np.testing.assert_allclose(b2, box, atol=1e-12)
    with pytest.raises(ValueError, match="atom types"):
        systems.read_structure(str(f), type_z=[8])


def test_npz_and_format_errors(tmp_path):
    pos, box, Z = _water()
    np.savez(tmp_path / "w.npz", pos=pos, box=box, Z=Z)
    p2, b2, z2 = systems.read_structure(str(tmp_path / "w.npz"))
    assert np.array_equal(p2, pos) and np.array_equal(z2, Z)
    tri = tmp_path / "t.xyz"
    tri.write_text('1\nLattice="10 0 0 1 10 0 0 0 10"\nH 0 0 0\n')
    with pytest.raises(ValueError, match="orthorhombic"):
        systems.read_structure(str(tri))
    nolat = tmp_path / "n.xyz"
    nolat.write_text("1\ncomment\nH 0 0 0\n")
    with pytest.raises(ValueError, match="Lattice"):
        systems.read_structure(str(nolat))
    unk = tmp_path / "u.xyz"
    unk.write_text('1\nLattice="10 0 0 0 10 0 0 0 10"\nXx 0 0 0\n')
    with pytest.raises(ValueError, match="unknown element"):
        systems.read_structure(str(unk))
    with pytest.raises(ValueError, match="formats"):
        systems.read_structure(str(tmp_path / "w.cif"))


def test_replica_atom_j_is_base_atom_j_mod_n():
    pos, box, Z = _water()
    pr, br, zr = systems.replicate(pos, box, Z, (2, 1, 3))
    n = len(pos)
    assert pr.shape == (6 * n, 3) and np.array_equal(br, box * [2, 1, 3]) and np.array_equal(zr, np.tile(Z, 6))
    j = np.arange(6 * n)
    shift = (pr - pos[j % n]) / box
    assert np.allclose(shift, np.round(shift), atol=1e-12)          # whole box lengths
    assert len({tuple(s) for s in np.round(shift).astype(int)}) == 6


def test_structure_options():
    import argparse
    ap = argparse.ArgumentParser()
    systems.add_structure_args(ap)
    pos, box, Z, base = systems.structure_from_args(ap.parse_args(["--water", "64", "--rep", "2", "1", "1"]))
    assert len(pos) == 2 * len(base[0]) and np.array_equal(box, base[1] * [2, 1, 1])
    with pytest.raises(SystemExit):
        ap.parse_args(["--water", "64", "--fcc", "3"])               # one source only
    with pytest.raises(ValueError, match="--rep"):
        systems.structure_from_args(ap.parse_args(["--structure", "x.xyz", "--rep", "2", "2", "2"]))


def test_element_tables():
    assert len(systems.SYMBOLS) == 89 and len(systems.MASS) == 89
    assert systems.SYMBOLS[0] == "H" and systems.SYMBOLS[7] == "O" and systems.SYMBOLS[25] == "Fe"
    # the benchmark species keep their masses (configuration 5's MD depends on them)
    assert systems.MASS[1] == 1.008 and systems.MASS[8] == 15.999 and systems.MASS[28] == 58.6934
    assert all(systems.MASS[z] < systems.MASS[z + 1] + 2 for z in range(1, 89))


@pytest.mark.parametrize("module", ["receiver_chunk_mace", "md"])
def test_command_lines_parse(module, capsys):
    import importlib
    main = importlib.import_module(f"mace_onegpu.{module}").main
    with pytest.raises(SystemExit) as e:
        main(["--help"])
    assert e.value.code == 0 and "--water" in capsys.readouterr().out
    with pytest.raises(SystemExit) as e:
        main(["--chunk", "100"])                                       # no structure
    assert e.value.code == 2
