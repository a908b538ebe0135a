"""The profile summaries' region split and kernel names, on a small database of the shape rocprofv3
writes (a `kernels` table of name, start, end in ns)."""
import sqlite3

from bybylang_amd import profile_summary as ps

MARK = "byhip::(anonymous namespace)::timing_mark(int)"
GEMV = ("void byhip::(anonymous namespace)::q4_gemv<1, 2, false, true, true, true, 1>"
        "(byhip::(anonymous namespace)::GemvArgs)")
SPLIT = "_ZN5byhip12_GLOBAL__N_114split_rows_f16EPKfiPiPDF16_S4_"


def make_db(path):
    rows, t = [], 0

    def add(name, dur, gap=100):
        nonlocal t
        rows.append((name, t, t + dur))
        t += dur + gap

    add(GEMV, 5000)  # before the first mark: in no region
    for region in range(4):
        add(MARK, 1000)
        for _ in range(3):
            add(GEMV, 7000 + 1000 * region)
        if region % 2:
            add(SPLIT, 4000)
        add(MARK, 1000)
        add(GEMV, 9000)  # between regions
    con = sqlite3.connect(path)
    con.execute("create table kernels (name text, start integer, end integer)")
    con.executemany("insert into kernels values (?, ?, ?)", rows)
    con.commit()
    con.close()
    return rows


def test_regions_split_at_mark_pairs(tmp_path):
    db = str(tmp_path / "k.db")
    rows = make_db(db)
    regs = ps.kernel_regions(db)
    assert len(regs) == 4
    marks = [(s, e) for n, s, e in rows if n == MARK]
    for i, (span, stats) in enumerate(regs):
        assert span == marks[2 * i + 1][0] - marks[2 * i][1]
        per = {name: (n, avg) for name, n, avg, _, _ in stats}
        assert per[GEMV] == (3, 7000 + 1000 * i)
        assert (SPLIT in per) == bool(i % 2)


def test_timed_table_keeps_every_second_region(tmp_path, capsys):
    db = str(tmp_path / "k.db")
    make_db(db)
    assert ps.main(["regions", db, "--timed"]) == 0
    lines = [l for l in capsys.readouterr().out.splitlines() if l.startswith("| ")]
    firsts = [l.split("|")[1].strip() for l in lines[1:]]
    assert firsts == ["1", "", "3", ""]
    assert "`q4_gemv<1, 2, false, true, true, true, 1>` | 3 | 8.000 |" in lines[1]
    assert "`split_rows_f16` | 1 | 4.000 |" in lines[2]


def test_short_names():
    assert ps.short_name(GEMV) == "q4_gemv<1, 2, false, true, true, true, 1>"
    assert ps.short_name(SPLIT) == "split_rows_f16"
    assert ps.short_name("(anonymous namespace)::read_words(HIP_vector_type<unsigned int, 4u> const*, "
                         "unsigned long, unsigned int*)") == "read_words"
    assert ps.short_name("byhip::(anonymous namespace)::q4_classify(float const*)") == "q4_classify"
