"""CPU parity oracle for the KV-cache attention path (test infrastructure only;
see oracle/oracle.py)."""
