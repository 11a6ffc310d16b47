"""CPU oracle for the TQ1_G128 path. Test infrastructure only; see ``tq1_oracle``."""
